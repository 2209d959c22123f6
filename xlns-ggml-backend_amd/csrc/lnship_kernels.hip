// gfx950 kernels of the LNS backend and their C ABI (include/lnship.h).
//
// Parallelism only ever spans independent outputs; every reduction (dot
// product, softmax normalizer, rms_norm sum of squares) runs in the
// reference's element order inside one lane (lns-backend/cuda/
// lns-cuda-kernels.h:16-21).  Weights are cached "k8-interleaved": element
// (k, m) of a K x M slice sits at ((k / 8) * M + m) * 8 + k % 8 with K padded
// to a multiple of 8, so one lane fetches eight consecutive k steps of its row
// in a single 16-byte load and a wave reads one contiguous 1 KiB block.
#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <type_traits>
#include <vector>

#include "lnship.h"
#include "lnship_device.h"
#include "lnship_tables.h"

namespace lnship {

constexpr int k_block = 256;
constexpr int k_max_devices = 64;
// LDS budget of a workgroup on gfx950 (160 KiB per CU)
constexpr int k_lds_bytes = 160 * 1024;
// what the row kernels' static shared arrays may take beside their dynamic LDS
constexpr int k_lds_static = 2048;
// The LDS copy of the xlns32 adder tables (32-bit words): 512 four-word
// descriptors of the interpolation, indexed by (opposite signs, binade of d),
// then -dlo, then dhi as pairs (two words per dh), then the interpolation
// tables sb, sbf (extended with zeros, and the exact-cancellation node, up
// to k32_co_cancel), db, dbf, and a zero pair.
constexpr int k32_desc_n = 512;
// the cotransformation's sentinels: e = (dh << 12) + dhi[dh] - dlo[dl] of
// the dh = 0 lanes starts at k32_co_h0, of the dl = 0 lanes at -dlo = k32_co_l0,
// so both fall in sbf's zeros; e of exact cancellation (d = 0) is their sum,
// the node that drives the sum below 0
constexpr uint32_t k32_co_h0 = 13u << 23, k32_co_l0 = 36u << 23;
constexpr uint32_t k32_co_cancel = k32_co_h0 + k32_co_l0;
constexpr int k32_sbf_ln = (int)((k32_co_cancel - k32_sb_end) >> k32_sb_fsh) + 2;   // LDS far-grid nodes: 594
constexpr int kl_desc = 0;
constexpr int kl_dlo = kl_desc + 4 * k32_desc_n;
constexpr int kl_dhi = kl_dlo + k32_co_n;
constexpr int kl_sb = kl_dhi + 2 * k32_co_n;
constexpr int kl_sbf = kl_sb + k32_sb_n;
constexpr int kl_db = kl_sbf + k32_sbf_ln;
constexpr int kl_dbf = kl_db + k32_db_n;
constexpr int kl_zero = kl_dbf + k32_db_fn;
constexpr int kl_end = (kl_zero + 4 + 3) & ~3;
constexpr int k_lds_tab32 = kl_end * 4;   // 134496 bytes
static_assert(kl_dlo % 4 == 0 && (kl_end - kl_dlo) % 4 == 0, "16-byte staging");
// The LDS image of the positive-sum adder (kernels whose only xlns32
// additions add positive values: rms_norm's sum of squares, soft_max's sum
// of exps): one (node, scaled slope) pair per grid interval of sb, the near
// grid's k32_sb_n - 1 intervals then the far grid's, extended with (0, 0)
// pairs from the essential zero to every distance below 2^31, so that no
// distance needs a cap.  A slope is
// t[i + 1] - t[i] scaled by 2^10 (near) or 2^9 (far): a 24-bit signed
// operand of v_mul_hi_i32_i24 whose product with the interval's fraction
// scaled by 2^9 (near) or 2^4 (far) has the floored interpolation term in
// its high word.
constexpr int kp32_near = k32_sb_n - 1;
constexpr int kp32_far = (int)((0x80000000u - k32_sb_end) >> k32_sb_fsh);
constexpr int kp32_pairs = (kp32_near + kp32_far + 1) & ~1;
constexpr int k_lds_pos32 = 8 * kp32_pairs;   // 129536 bytes
constexpr int kp32_near_slope = 10, kp32_near_frac = 9, kp32_far_slope = 9, kp32_far_frac = 4;
static_assert(kp32_near_slope + kp32_near_frac == 32 - k32_sb_sh, "near interpolation scale");
static_assert(kp32_far_slope + kp32_far_frac == 32 - k32_sb_fsh, "far interpolation scale");
static_assert((k32_sb_end & ((1u << k32_sb_fsh) - 1)) == 0, "the far grid starts on a far node");

static thread_local std::string t_err;

static int fail(int code, const char *fmt, const char *what = "") {
    char buf[256];
    std::snprintf(buf, sizeof buf, fmt, what);
    t_err = buf;
    return code;
}

static int hip_fail(hipError_t e, const char *where) {
    char buf[256];
    std::snprintf(buf, sizeof buf, "%s: %s", where, hipGetErrorString(e));
    t_err = buf;
    return LNSHIP_EDEVICE;
}

#define LNSHIP_HIP(call)                                          \
    do {                                                          \
        hipError_t e_ = (call);                                   \
        if (e_ != hipSuccess) return hip_fail(e_, #call);         \
    } while (0)

// ---- per-device state -----------------------------------------------------

struct device_state {
    bool ready = false;
    int cus = 0;   // compute units
    dev_tables T{};
    void *scratch = nullptr;   // grow-only
    size_t scratch_size = 0;
    std::vector<void *> retired;   // outgrown scratch blocks, kept for captured graphs
    void *fixed_scratch = nullptr;  // this device's copy of `scratch` (below), from hipGetSymbolAddress
    // index check of get_rows / set_rows: [0] set to 1 by the first
    // out-of-range index since the last lnship_index_error, [1] that index
    unsigned long long *index_err = nullptr;
};

static device_state g_devices[k_max_devices];

// The activation staging of lnship32_mul_mat_noalloc: a fixed block in the
// code object, so that entry point allocates nothing.  Every GPU the library
// runs on holds its own copy until the process ends.  In host code this
// name is not a device address: host code uses device_state::fixed_scratch,
// which lnship_init sets from hipGetSymbolAddress on each device.
constexpr size_t k_fixed_scratch_bytes = (size_t)4 << 20;
static __device__ __align__(256) unsigned char scratch[k_fixed_scratch_bytes];
static std::mutex g_mutex;
static host_tables *g_host = nullptr;

static int current_device(int *dev) {
    LNSHIP_HIP(hipGetDevice(dev));
    if (*dev < 0 || *dev >= k_max_devices) return fail(LNSHIP_EDEVICE, "device index out of range%s");
    return 0;
}

template <class T>
static int upload(const T *src, size_t n, const T **dst) {
    void *p = nullptr;
    LNSHIP_HIP(hipMalloc(&p, n * sizeof(T)));
    LNSHIP_HIP(hipMemcpy(p, src, n * sizeof(T), hipMemcpyHostToDevice));
    *dst = static_cast<const T *>(p);
    return 0;
}

static device_state *state() {
    int dev = 0;
    if (current_device(&dev) != 0) return nullptr;
    device_state *s = &g_devices[dev];
    if (!s->ready) {
        fail(LNSHIP_ENOINIT, "lnship_init was not called for this device%s");
        return nullptr;
    }
    return s;
}

// Grow-only device scratch of the current device; callers on one device are
// serialized by the stream order of their launches.  A HIP graph captured
// earlier keeps the address it was captured with, so a block that is
// outgrown is retired, never freed: it stays valid for such graphs until the
// process ends (the sizes at least double, so the retired blocks together
// are smaller than the live one).  Growing while the stream is capturing
// would put an allocation inside the capture, so it is refused: the caller
// runs the op once outside the capture first.
static int grow_scratch(device_state *s, size_t bytes, void **p, hipStream_t st) {
    std::lock_guard<std::mutex> lock(g_mutex);
    if (bytes > s->scratch_size) {
        hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
        LNSHIP_HIP(hipStreamIsCapturing(st, &cs));
        if (cs != hipStreamCaptureStatusNone)
            return fail(LNSHIP_ERANGE, "device scratch would grow inside a HIP graph capture (run the op once "
                                       "before capturing it)%s");
        size_t sz = std::max({bytes, (size_t)1 << 20, 2 * s->scratch_size});
        void *q = nullptr;
        LNSHIP_HIP(hipMalloc(&q, sz));
        if (s->scratch) s->retired.push_back(s->scratch);
        s->scratch = q;
        s->scratch_size = sz;
    }
    *p = s->scratch;
    return 0;
}

static unsigned grid_for(int64_t n, int per_thread = 1) {
    int64_t b = (n + (int64_t)k_block * per_thread - 1) / ((int64_t)k_block * per_thread);
    return (unsigned)std::max<int64_t>(1, std::min<int64_t>(b, 65535));
}

// ---- LFSR jump-ahead --------------------------------------------------------

__device__ __forceinline__ uint32_t lfsr_jump(const dev_tables &T, uint32_t s, uint64_t n) {
    if (s == 0) return 0;
    uint32_t i = T.lfsr_log[s];
    return T.lfsr_seq[(uint32_t)(((uint64_t)i + n % 65535u) % 65535u)];
}

// ---- conversions ------------------------------------------------------------

__global__ void k_from_f32_16(const float *__restrict__ src, uint16_t *__restrict__ dst, int64_t n,
                              const uint16_t *__restrict__ cvt) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x)
        dst[i] = (uint16_t)x16_from_f32(cvt, src[i]);
}

__global__ void k_to_f32_16(const uint16_t *__restrict__ src, float *__restrict__ dst, int64_t n,
                            const float *__restrict__ rev) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x)
        dst[i] = rev[src[i]];
}

__global__ void k_from_f32_32(const float *__restrict__ src, uint32_t *__restrict__ dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x)
        dst[i] = x32_from_f32(src[i]);
}

__global__ void k_to_f32_32(const uint32_t *__restrict__ src, float *__restrict__ dst, int64_t n) {
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x)
        dst[i] = x32_to_f32(src[i]);
}

__device__ __forceinline__ float load_elem(const void *src, int is_f16, int64_t i) {
    if (is_f16) return __half2float(reinterpret_cast<const __half *>(src)[i]);
    return reinterpret_cast<const float *>(src)[i];
}

// rows x cols row-major -> k8-interleaved (k = col, m = row), one slice per
// blockIdx.y; padding columns (cols..Kp) get code 0.
template <int W32>
__global__ void k_pack(const void *__restrict__ src, int src_type, int64_t src_ld, int64_t src_slice,
                       void *__restrict__ dst, int64_t rows, int64_t cols, int64_t kp,
                       const uint16_t *__restrict__ cvt) {
    const int64_t n = rows * kp;
    const int64_t z = blockIdx.y;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        const int64_t r = i / kp, c = i - r * kp;
        const int64_t o = z * rows * kp + ((c >> 3) * rows + r) * 8 + (c & 7);
        const bool pad = c >= cols;
        const int64_t at = z * src_slice + r * src_ld + c;
        if (!W32 && src_type == 2) {   // xlns16 codes, taken as they are
            reinterpret_cast<uint16_t *>(dst)[o] = pad ? (uint16_t)0 : reinterpret_cast<const uint16_t *>(src)[at];
            continue;
        }
        float v = 0.0f;
        if (!pad) v = load_elem(src, src_type, at);
        if (W32) reinterpret_cast<uint32_t *>(dst)[o] = pad ? 0u : x32_from_f32(v);
        else reinterpret_cast<uint16_t *>(dst)[o] = pad ? (uint16_t)0 : (uint16_t)x16_from_f32(cvt, v);
    }
}

// activation rows (N per slice, row stride x_ld, slice stride x_slice) into
// contiguous padded LNS rows [slice][N][Kp]
template <int W32>
__global__ void k_act(const float *__restrict__ x, int64_t x_ld, int64_t x_slice, void *__restrict__ dst,
                      int64_t N, int64_t K, int64_t kp, const uint16_t *__restrict__ cvt) {
    const int64_t n_all = N * kp;
    const int64_t z = blockIdx.y;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n_all; i += (int64_t)blockDim.x * gridDim.x) {
        const int64_t r = i / kp, c = i - r * kp;
        const int64_t o = z * n_all + i;
        if (c >= K) {
            if (W32) reinterpret_cast<uint32_t *>(dst)[o] = 0u;
            else reinterpret_cast<uint16_t *>(dst)[o] = 0;
            continue;
        }
        const float v = x[z * x_slice + r * x_ld + c];
        if (W32) reinterpret_cast<uint32_t *>(dst)[o] = x32_from_f32(v);
        else reinterpret_cast<uint16_t *>(dst)[o] = (uint16_t)x16_from_f32(cvt, v);
    }
}

// ---- reductions -------------------------------------------------------------
// One accumulator per (row, column) per lane; start / add / finish as in the
// reference's reduction policies (cuda/lns-cuda-xlns16.cu:67-130).  The
// accumulator keeps its log field and its sign in separate registers, so the
// dependent chain of one addition is |dlog| -> table index -> LDS read ->
// add -> clamp; the sign and the exact-cancellation case run beside it.
// Exact cancellation (equal logs, opposite signs) reads a sentinel table
// entry that clamps the log to 0 and forces the sign to +.

// |a - b| as one v_sad_u32 (max - min + z, z = 0 held in a register)
__device__ __forceinline__ uint32_t absdiff(uint32_t a, uint32_t b, uint32_t z) { return max(a, b) - min(a, b) + z; }
__device__ __forceinline__ uint32_t absdiff(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_sad_u32 %0, %1, %2, 0" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

__device__ __forceinline__ int32_t mul_i24(int32_t a, int32_t b) {
    int32_t r;
    asm("v_mul_i32_i24 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// Packed 16-bit integer operations on both halves of a register: a - b
// with unsigned saturation at 0, and the unsigned minimum (v_pk_sub_u16 with
// clamp, v_pk_min_u16).
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_sub_sat_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_sub_sat(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}
__device__ __forceinline__ uint32_t pk_min_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_min(__builtin_bit_cast(u16x2, a), __builtin_bit_cast(u16x2, b)));
}
// Both halves: a - b wrapping (v_pk_sub_u16); and a + b with signed
// saturation, then at least 0 (v_pk_add_i16 with clamp, v_pk_max_i16).
typedef short i16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pk_sub_u16(uint32_t a, uint32_t b) {
    return __builtin_bit_cast(uint32_t, __builtin_bit_cast(u16x2, a) - __builtin_bit_cast(u16x2, b));
}
__device__ __forceinline__ uint32_t pk_add_sat_nonneg_i16(uint32_t a, uint32_t b) {
    const i16x2 s = __builtin_elementwise_add_sat(__builtin_bit_cast(i16x2, a), __builtin_bit_cast(i16x2, b));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(s, i16x2{0, 0}));
}

// Shift-adds in plain code select to one v_lshl_add_u32 each.  The lds_at
// forms are the same instruction in inline asm, used where an LDS read is
// the only reader: the compiler keeps them whole (as plain code it splits a
// masked index into shift, mask and add), and an LDS read has no forwarding
// hazard on an inline asm result (a vector ALU reader would get a wait state).
__device__ __forceinline__ uint32_t lshl2_add(uint32_t a, uint32_t b) { return (a << 2) + b; }
__device__ __forceinline__ uint32_t lshl3_add(uint32_t a, uint32_t b) { return (a << 3) + b; }
__device__ __forceinline__ uint32_t lds_at2(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_lshl_add_u32 %0, %1, 2, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t lds_at3(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_lshl_add_u32 %0, %1, 3, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t lds_at4(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_lshl_add_u32 %0, %1, 4, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}

// (a & m) | (b & ~m): a select on a lane mask held in a vector register,
// with no compare and no condition register (whose write and read would
// need hazard wait states on gfx950)
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) { return (a & m) | (b & ~m); }

// All ones where x is negative as a signed value, else 0, as one v_bfe_i32
// of bit 31 whose width comes from a register (one = 1 in a register the
// compiler cannot see into).  A plain shift would be folded into a compare
// and a select through the condition register.
__device__ __forceinline__ uint32_t sign_mask(uint32_t x, uint32_t one) {
    return (uint32_t)__builtin_amdgcn_sbfe((int32_t)x, 31, one);
}

// LDS addresses as 32-bit integers: a table lookup is then a shift-add of the
// index onto a precomputed origin and the read itself, with no separate add
// of the shared-memory base on the dependent chain.
typedef const int32_t __attribute__((address_space(3))) *lds_i32_t;
__device__ __forceinline__ uint32_t lds_addr(const void *p) { return (uint32_t)(uintptr_t)(lds_i32_t)p; }
__device__ __forceinline__ int32_t lds_ld(uint32_t addr) { return *(lds_i32_t)(uintptr_t)addr; }
// two or four consecutive words in one LDS read (ds_read_b64, ds_read_b128)
typedef int32_t i32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef const i32x2 __attribute__((address_space(3))) *lds_i2_t;
typedef const u32x4 __attribute__((address_space(3))) *lds_u4_t;
__device__ __forceinline__ i32x2 lds_ld2(uint32_t addr) { return *(lds_i2_t)(uintptr_t)addr; }
__device__ __forceinline__ u32x4 lds_ld4(uint32_t addr) { return *(lds_u4_t)(uintptr_t)addr; }

struct acc_ls {
    uint32_t l, s;   // log field, sign bit in place
};

template <int MODE>
struct red16;

template <>
struct red16<LNSHIP_BASE> {
    const char *g;   // LDS: (sb, db) int16 pairs per distance d <= esszer + 1
    using acc_t = acc_ls;
    __device__ __forceinline__ acc_t start(uint32_t v, uint32_t &) const { return {v & k16_logmask, v & k16_sign}; }
    __device__ __forceinline__ void add_ls(acc_t &a, uint32_t tl, uint32_t ts, uint32_t &) const {
        const uint32_t d = absdiff(a.l, tl), mx = max(a.l, tl);
        const uint32_t usedb = a.s ^ ts;
        // the sign picks the pair half off the critical path: the address is
        // then one shift-add of the clamped distance
        const char *gs = g + (usedb >> 14);
        const int32_t adj = *reinterpret_cast<const int16_t *>(gs + (min(d, (uint32_t)k16_esszer + 1) << 2));
        const uint32_t ns = a.l > tl ? a.s : ts;
        a.l = (uint32_t)min(max((int32_t)mx + adj, 0), (int32_t)k16_logmask);
        a.s = (d == 0 && usedb) ? 0u : ns;
    }
    __device__ __forceinline__ void add(acc_t &a, uint32_t v, uint32_t &st) const { add_ls(a, v & k16_logmask, v & k16_sign, st); }
    // add() of a positive v to a positive sum (sums of squares, of exps): sb
    // only, the sign stays +
    __device__ __forceinline__ void add_pos(acc_t &a, uint32_t v, uint32_t &) const {
        const uint32_t tl = v & k16_logmask;
        const uint32_t d = absdiff(a.l, tl), mx = max(a.l, tl);
        const int32_t adj = *reinterpret_cast<const int16_t *>(g + (min(d, (uint32_t)k16_esszer + 1) << 2));
        a.l = (uint32_t)min(max((int32_t)mx + adj, 0), (int32_t)k16_logmask);
    }
    __device__ __forceinline__ uint32_t finish(const acc_t &a) const { return a.s | a.l; }
};

template <>
struct red16<LNSHIP_MONTE> {
    const int32_t *gm;   // LDS: (sb e, sb m, db e, db m) per distance
    uint32_t gb;         // gm's LDS byte address
    using acc_t = acc_ls;
    __device__ __forceinline__ acc_t start(uint32_t v, uint32_t &) const { return {v & k16_logmask, v & k16_sign}; }
    // One LFSR step; below the dither range the base table's adjustment, from
    // it on one ulp toward the smaller operand with probability F(d)/64,
    // decided by the top 6 bits r of the new state: sb adds (F + r) >> 6,
    // db (64 - F + ~r) >> 6, here (-F + (63 - r)) >> 6 from the image's
    // (-F, 63).  The larger log is added scaled by 64 in the same add, so
    // after the table read only a mask, an add, a shift and the clamp remain.
    // The sign: the larger operand's (bit 15 of tl - a.l is set iff a.l >
    // tl), + for exact cancellation (bit 15 of d - 1 is set iff d = 0).
    __device__ __forceinline__ void add_ls(acc_t &a, uint32_t tl, uint32_t ts, uint32_t &st) const {
        st = lfsr_step(st);
        const uint32_t d = absdiff(a.l, tl), mx = max(a.l, tl);
        const uint32_t usedb = a.s ^ ts;   // 0 or k16_sign
        // row min(d, end) of 16 bytes, db's pair 8 bytes in
        const i32x2 em = lds_ld2(lds_at4(min(d, (uint32_t)k16_mc_end), gb + (usedb >> 12)));
        // the draw r, or 63 - r for db (r xor all ones under the mask 63)
        const uint32_t x = ((st >> 10) ^ (uint32_t)((int32_t)(usedb << 16) >> 31)) & (uint32_t)em.y;
        const int32_t sum = (int32_t)(mx << 6) + em.x + (int32_t)x;
        a.s = bfi(tl - a.l, a.s, ts) & ~(usedb & (d - 1u));
        a.l = (uint32_t)min(max(sum >> 6, 0), (int32_t)k16_logmask);
    }
    __device__ __forceinline__ void add(acc_t &a, uint32_t v, uint32_t &st) const { add_ls(a, v & k16_logmask, v & k16_sign, st); }
    // add() of a positive v to a positive sum: sb's half of the row, no
    // sign work (the same draws)
    __device__ __forceinline__ void add_pos(acc_t &a, uint32_t v, uint32_t &st) const {
        st = lfsr_step(st);
        const uint32_t tl = v & k16_logmask;
        const uint32_t d = absdiff(a.l, tl), mx = max(a.l, tl);
        const i32x2 em = lds_ld2(lds_at4(min(d, (uint32_t)k16_mc_end), gb));
        const int32_t sum = (int32_t)(mx << 6) + em.x + (int32_t)((st >> 10) & (uint32_t)em.y);
        a.l = (uint32_t)min(max(sum >> 6, 0), (int32_t)k16_logmask);
    }
    __device__ __forceinline__ uint32_t finish(const acc_t &a) const { return a.s | a.l; }
};

// xlns32 addition (xlns32_alt), branch-free.  The Gaussian log at distance
// d has three exclusive cases: sb(d) for equal signs; db(d) from its tables
// at and above 2 binades; below 2 binades the cotransformation
//   1 - 2^-d = (1 - 2^-dh) + 2^-dh (1 - 2^-dl),  d = (dh << 12) + dl,
// which is dlo[dl] when dh = 0, dhi[dh] when dl = 0, and otherwise
// dhi[dh] + sb(e) with e = (dh << 12) - dlo[dl] + dhi[dh].  A lane needs at
// most one interpolation (at e on the sb tables, or at d on the sb / db
// tables), so all lanes share one.  T is the LDS copy of the adder tables
// (lds32_image): dlo negated (with a sentinel at dl = 0), dhi as pairs
// ((dh << 12) + dhi[dh], -dhi[dh]) (with sentinels at dh = 0), so that e is
// one add and the addend outside the interpolation, max(dhi, dlo) on
// cotransformation lanes and 0 elsewhere, is the negated minimum of the
// pair's second word, -dlo and the descriptor's cap; sbf runs on in zeros
// past the essential zero to the node of exact cancellation.  Every select
// is arithmetic: a ternary around two table reads would compile to a
// divergent branch that serialises both.

// Byte offsets of the interpolation tables in the LDS copy, each less its
// grid origin, so that a distance x on grid shift sh reads node
// (x >> sh) at origin + ((x >> sh) << 2).
constexpr uint32_t kb_sb = (uint32_t)kl_sb * 4;
constexpr uint32_t kb_sbf = (uint32_t)(kl_sbf - (int)(k32_sb_end >> k32_sb_fsh)) * 4;
constexpr uint32_t kb_db = (uint32_t)(kl_db - k32_db_first) * 4;
constexpr uint32_t kb_dbf = (uint32_t)(kl_dbf - (int)(k32_db_end >> k32_db_fsh)) * 4;

// LDS byte addresses of the adder's tables (interpolation tables less their
// grid origin), computed once per kernel; the empty asm keeps them opaque
// registers, so that picking a table is one select and no base add follows.
struct x32_tab {
    uint32_t dlo, dhi, sb, sbf, db, dbf, zero, desc;
    uint32_t one;   // 1 in a register the compiler cannot see into
    // a mask and a bound in registers: two-operand instructions take them in
    // their short encoding (a literal operand makes an instruction 8 bytes)
    uint32_t m0fff, ksb;
};
__device__ __forceinline__ x32_tab x32_origins(const int32_t *T) {
    uint32_t tb = lds_addr(T);
    asm("" : "+v"(tb));
    x32_tab o{tb + (uint32_t)kl_dlo * 4, tb + (uint32_t)kl_dhi * 4, tb + kb_sb, tb + kb_sbf, tb + kb_db,
              tb + kb_dbf, tb + (uint32_t)kl_zero * 4, tb + (uint32_t)kl_desc * 4, 1u, 0xfffu, k32_sb_end - 1u};
    // each origin its own register: a select among them stays a select (not
    // a lookup table of their constant offsets)
    asm("" : "+v"(o.sb), "+v"(o.sbf), "+v"(o.db), "+v"(o.dbf), "+v"(o.zero), "+v"(o.one));
    asm("" : "+v"(o.m0fff), "+v"(o.ksb));
    return o;
}


// The same addition ordered for one chain per lane, where every instruction
// of the wave is on the chain's clock (a single wave issues about one
// instruction per 2 ns).  Two rounds of LDS lookups.  First a descriptor
// keyed by (opposite signs, binade of d), the cotransformation's -dlo[dl] and
// the dhi pair of dh; then the pair of grid nodes around x, where x is d on
// the sb / db grid the descriptor names (the zero pair from the essential
// zero on), or, on cotransformation lanes, e on sb's near or far grid.  The
// dl = 0 and dh = 0 sentinels put e beyond the essential zero, where the sb
// tables read 0, so every cotransformation lane interpolates at e and adds
// dlo[dl] (dh = 0) or dhi[dh] besides.  The selects are bit-field inserts on
// lane masks from the descriptor or from sign bits, with no compare.  The
// larger log, the result's sign and the caller's `shadow` work (the next
// product) fill the first round trip; what the tail needs the second.
// Scheduling barriers keep the groups in this order.
// One addition of a single-chain step: a <- a (+) (tl, ts).  u = a.s ^ ts
// (the opposite-signs flag, bit 31); shadow() runs in the first round trip
// and returns the next addend's sign nts; post() runs in the second.
// Returns the next step's flag, the new a.s ^ nts.
template <class F, class P>
__device__ __forceinline__ uint32_t x32_add_step(const x32_tab &O, acc_ls &a, uint32_t tl, uint32_t ts, uint32_t u,
                                                 F &&shadow, P &&post) {
    // du = |a.l - tl| + u: d with the opposite-signs flag in bit 31, in one
    // v_sad_u32; its fields index the three reads, and the descriptors of
    // opposite-sign keys carry origins less 2^31 >> shift (x = du there)
    const uint32_t du = absdiff(a.l, tl, u);
    // the three addresses after the three indices, in one asm block so that
    // each shift-add waits on an index formed two instructions earlier: the
    // reads of -dlo[dl], of the dhi pair of dh ((dh << 12) + dhi[dh], -dhi[dh],
    // or the sentinels for dh = 0) and of the descriptor (origin, grid shift,
    // cap of e, cotransformation lane mask) go out back to back
    uint32_t a_lo, a_hi, a_ds;
    asm("v_lshl_add_u32 %0, %3, 2, %6\n\tv_lshl_add_u32 %1, %4, 3, %7\n\tv_lshl_add_u32 %2, %5, 4, %8"
        : "=&v"(a_lo), "=&v"(a_hi), "=&v"(a_ds)
        : "v"(du & O.m0fff), "v"(__builtin_amdgcn_ubfe(du, k32_co_sh, k32_co_sh)), "v"(du >> 23), "v"(O.dlo),
          "v"(O.dhi), "v"(O.desc));
    const int32_t lo = lds_ld(a_lo);
    const i32x2 hp = lds_ld2(a_hi);
    const u32x4 dsc = lds_ld4(a_ds);
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t mx = max(a.l, tl);
    // sign: the larger operand's (bit 31 of tl - a.l is set when a.l > tl),
    // and + for exact cancellation (with u set, bit 31 of du - 1 is clear
    // only for d = 0)
    const uint32_t nsign = bfi(tl - a.l, a.s, ts) & (~u | (du - 1u));
    const uint32_t un = nsign ^ shadow();
    // formed here, in the first round trip
    asm volatile("" ::"v"(mx), "v"(nsign), "v"(un));
    __builtin_amdgcn_sched_barrier(0);
    // k = ksb - e (this image's dhi pairs hold ksb - th2); x: e on
    // cotransformation lanes, du elsewhere; the far grid where k < 0 on
    // cotransformation lanes (lane mask -1) and never elsewhere (mask 0)
    const uint32_t k = (uint32_t)hp.x - (uint32_t)lo;
    const uint32_t x = bfi(dsc.w, O.ksb - k, du);
    const uint32_t hi = sign_mask((uint32_t)max((int32_t)k, (int32_t)dsc.w), O.one);
    const uint32_t sh = bfi(hi, (uint32_t)k32_sb_fsh, dsc.y);
    const uint32_t node = lshl2_add(x >> sh, bfi(hi, O.sbf, dsc.x));
    const int32_t t0 = lds_ld(node), t1 = lds_ld(node + 4);
    __builtin_amdgcn_sched_barrier(0);
    // the addend outside the interpolation, less: -dlo[dl] where dh = 0,
    // else -dhi[dh] (the smaller of the two) on cotransformation lanes, and
    // the cap 0 elsewhere
    const int32_t mA = (int32_t)mx - (int32_t)min(min((uint32_t)hp.y, (uint32_t)lo), dsc.z);
    const int32_t frac = (int32_t)__builtin_amdgcn_ubfe(x, 0, sh);
    post();
    __builtin_amdgcn_sched_barrier(0);
    const int32_t ip = t0 + (__mul24(t1 - t0, frac) >> sh);
    a.l = (uint32_t)max(__builtin_elementwise_add_sat(mA, ip), 0);
    a.s = nsign;
    return un;
}

// One addition of a chain, u computed here (one dependent step more)
template <class F>
__device__ __forceinline__ void x32_add_desc(const x32_tab &O, acc_ls &a, uint32_t tl, uint32_t ts, F &&shadow) {
    x32_add_step(
        O, a, tl, ts, a.s ^ ts,
        [&] {
            shadow();
            return 0u;
        },
        [] {});
}

// x32_add_desc without the scheduling order, for lanes that run several
// chains (the compiler interleaves them)
__device__ __forceinline__ void x32_add_ls(const x32_tab &O, acc_ls &a, uint32_t tl, uint32_t ts) {
    const uint32_t u = a.s ^ ts;
    const uint32_t du = absdiff(a.l, tl, u);
    const int32_t lo = lds_ld(lds_at2(du & ((1u << k32_co_sh) - 1u), O.dlo));
    const i32x2 hp = lds_ld2(lds_at3(__builtin_amdgcn_ubfe(du, k32_co_sh, k32_co_sh), O.dhi));
    const u32x4 dsc = lds_ld4(lds_at4(du >> 23, O.desc));
    const uint32_t mx = max(a.l, tl);
    const uint32_t nsign = bfi(tl - a.l, a.s, ts) & (~u | (du - 1u));
    const uint32_t xe = min((uint32_t)hp.x + (uint32_t)lo, dsc.z);
    const uint32_t x = bfi(dsc.w, xe, du);
    const bool far = xe > k32_sb_end - 1u;
    const uint32_t sh = far ? (uint32_t)k32_sb_fsh : dsc.y;
    const uint32_t node = lshl2_add(x >> sh, far ? O.sbf : dsc.x);
    const int32_t t0 = lds_ld(node), t1 = lds_ld(node + 4);
    const int32_t mA = (int32_t)mx - (int32_t)min(min((uint32_t)hp.y, (uint32_t)lo), dsc.z);
    const int32_t frac = (int32_t)__builtin_amdgcn_ubfe(x, 0, sh);
    const int32_t ip = t0 + (__mul24(t1 - t0, frac) >> sh);
    a.l = (uint32_t)max(__builtin_elementwise_add_sat(mA, ip), 0);
    a.s = nsign;
}

// An xlns32 addition of two positive values, for sums whose every addend is
// positive (sums of squares, sums of exps): the sign stays +, the adjustment
// is always sb(d), and one round of LDS reads suffices, the node pair around
// d on sb's near or far grid.  d is capped at the essential zero, where the
// far grid's last node and the interpolation read 0.  The result needs no
// clamp at 0 (sb >= 0); it saturates on overflow as the general addition.
__device__ __forceinline__ uint32_t x32_add_pos(const x32_tab &O, uint32_t al, uint32_t tl) {
    // (the explicit v_sad_u32: from max - min + 0 the compiler makes four
    // instructions here, all on the chain)
    const uint32_t xd = min(absdiff(al, tl), k32_esszer);
    const uint32_t hi = sign_mask(k32_sb_end - 1u - xd, O.one);   // d on the far grid
    const uint32_t sh = bfi(hi, (uint32_t)k32_sb_fsh, (uint32_t)k32_sb_sh);
    const uint32_t node = lshl2_add(xd >> sh, bfi(hi, O.sbf, O.sb));
    const int32_t t0 = lds_ld(node), t1 = lds_ld(node + 4);
    const int32_t mx = (int32_t)max(al, tl);
    const int32_t frac = (int32_t)__builtin_amdgcn_ubfe(xd, 0, sh);
    const int32_t ip = t0 + (__mul24(t1 - t0, frac) >> sh);
    return (uint32_t)__builtin_elementwise_add_sat(mx, ip);
}

// The positive-sum addition over the pair image (k_lds_pos32): the same
// result as x32_add_pos in fewer dependent operations.  The addresses of
// both grids' pairs are formed side by side and one is picked by the far
// mask; the interpolation term is the high word of one 24-bit multiply of
// the stored scaled slope and the scaled fraction (formed while the read is
// in flight), so after the read only that multiply and two adds remain.
struct pos_tab {
    uint32_t near, far;   // LDS byte addresses: near pairs, far pairs less the far grid's origin
    uint32_t one, zero;   // 1 and 0 in registers the compiler cannot see into
};
__device__ __forceinline__ int32_t sext24(uint32_t x) { return (int32_t)(x << 8) >> 8; }
// On one wave every instruction is on the chain's clock, so the read is
// issued after the seven instructions that form its address (the distance,
// the far mask, the grid's shift and origin, the shift-add), and the
// fraction and the larger log are formed in its shadow (scheduling barriers
// keep that order: left alone the compiler forms the fraction first).
__device__ __forceinline__ uint32_t x32_add_pos2(const pos_tab &P, uint32_t al, uint32_t tl) {
    const uint32_t d = absdiff(al, tl, P.zero);   // one v_sad_u32; < 2^31: the far pairs reach every distance
    const uint32_t far = sign_mask(k32_sb_end - 1u - d, P.one);   // d on the far grid
    const uint32_t sh = bfi(far, (uint32_t)k32_sb_fsh, (uint32_t)k32_sb_sh);
    const i32x2 tp = lds_ld2(lds_at3(d >> sh, bfi(far, P.far, P.near)));
    __builtin_amdgcn_sched_barrier(0);
    const uint32_t fr = __builtin_amdgcn_ubfe(d, 0, sh) << bfi(far, (uint32_t)kp32_far_frac, (uint32_t)kp32_near_frac);
    const int32_t mx = (int32_t)max(al, tl);
    asm volatile("" ::"v"(fr), "v"(mx));
    __builtin_amdgcn_sched_barrier(0);
    // the high word of the product of two 24-bit signed operands (one
    // v_mul_hi_i32_i24): both fit, so the sign extensions are free
    const int32_t q = (int32_t)(((int64_t)sext24((uint32_t)tp.y) * (int64_t)sext24(fr)) >> 32);
    return (uint32_t)__builtin_elementwise_add_sat(mx, tp.x + q);
}

// A whole xlns32 addition on packed values (sign bit 31) over the LDS tables.
__device__ __forceinline__ uint32_t x32_add_lds(const x32_tab &O, uint32_t x, uint32_t y) {
    acc_ls a{x & k32_logmask, x & k32_sign};
    x32_add_ls(O, a, y & k32_logmask, y & k32_sign);
    return a.s | a.l;
}

template <>
struct red16<LNSHIP_SUM32> {
    x32_tab O;
    using acc_t = acc_ls;   // xlns32: 31-bit log, sign in bit 31
    __device__ __forceinline__ acc_t start(uint32_t v, uint32_t &) const {
        return {(v & k16_logmask) << 16, (v & k16_sign) << 16};
    }
    __device__ __forceinline__ void add_ls(acc_t &a, uint32_t tl, uint32_t ts, uint32_t &) const {
        x32_add_ls(O, a, tl << 16, ts << 16);
    }
    // operands already widened (log and sign moved to the xlns32 positions)
    template <class F>
    __device__ __forceinline__ void add_lat(acc_t &a, uint32_t tl32, uint32_t ts32, F &&shadow) const {
        x32_add_desc(O, a, tl32, ts32, shadow);
    }
    __device__ __forceinline__ void add(acc_t &a, uint32_t v, uint32_t &st) const { add_ls(a, v & k16_logmask, v & k16_sign, st); }
    __device__ __forceinline__ uint32_t finish(const acc_t &a) const {
        const uint32_t s = a.s | a.l;
        if (a.l >= 0x7fff8000u) return (s >> 16) | k16_logmask;
        return (s + 0x8000u) >> 16;
    }
};

// LPVIP: ROM-less xlns32 adder (Mitchell antilog + corrected Mitchell log;
// the exact Gaussian log within one binade of the db singularity).
// The low 32 bits and bits 32-47 of the product of two 24-bit operands
// (v_mul_u32_u24, v_mul_hi_u32_u24: full rate, where a 64-bit product takes
// a quarter-rate multiply-add)
__device__ __forceinline__ uint32_t mul_u24(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_mul_u32_u24 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t mulhi_u24(uint32_t a, uint32_t b) {
    uint32_t r;
    asm("v_mul_hi_u32_u24 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
    return r;
}
__device__ __forceinline__ uint32_t mitchell_exp2_neg(uint32_t d) {
    uint32_t q = d >> 23, r = d & 0x7fffffu;
    if (q >= 31) return 0;
    return ((0x1000000u - r) >> 1) >> q;
}
__device__ __forceinline__ int32_t lpvip_sb(uint32_t d) {
    uint32_t u = mitchell_exp2_neg(d);
    uint64_t corr = ((uint64_t)u * (uint64_t)(0x800000u - u)) >> 23;
    return (int32_t)(u + (uint32_t)((corr * 0x2B8u) >> 11));
}
// The reference's round(2^23 log(1 - pow(2, -x)) / log(2)), x = d / 2^23,
// for 0 < d < 2^23, from tables (lp: host_tables::lpdb): 2^-x as
// 2^(-k/256) e^(-r ln 2) (r < 1/256, Taylor to degree 5), y = 1 - 2^-x with
// one rounding, then log2 y as e + log2(1 + j/256) + log2(1 + s) with
// s = m / (1 + j/256) - 1 < 2^-8 (degree 6); the polynomials by Estrin's
// scheme.  About half the dependent FP64 latency of log2(1 - exp2(-x)) with
// the library's functions, and the same integer for every d (every one of
// the 2^23 - 1 checked on the GPU against the oracle); contraction is off, so
// every caller compiles the same operations.
__device__ __forceinline__ int32_t lpvip_db_near(const double *lp, uint32_t d) {
#pragma clang fp contract(off)
    const double *E = lp, *IV = lp + k_lp_n, *LG = lp + 2 * k_lp_n;
    const double z = (double)(d & 0x7fffu) * (-0.69314718055994530942 / 8388608.0);   // -r ln 2
    const double z2 = z * z;
    const double pa = fma(z, 1.0 / 6.0, 0.5), pb = fma(z, 1.0 / 120.0, 1.0 / 24.0);
    const double p = fma(z2, fma(z2, pb, pa), 1.0 + z);
    const double y = fma(-E[d >> 15], p, 1.0);
    const int e = __builtin_amdgcn_frexp_exp(y);                    // y = m 2^e, m in [0.5, 1)
    const double m2 = __builtin_amdgcn_frexp_mant(y) * 2.0;         // [1, 2)
    const uint32_t j = (uint32_t)(__double2hiint(m2) >> 12) & 255u; // its top 8 mantissa bits
    const double sv = fma(m2, IV[j], -1.0);                          // [0, 2^-8)
    constexpr double c = 1.4426950408889634074;                      // 1 / ln 2
    const double s2 = sv * sv;
    const double u0 = fma(sv, -c / 2.0, c), u1 = fma(sv, -c / 4.0, c / 3.0), u2 = fma(sv, -c / 6.0, c / 5.0);
    const double h = fma(s2, fma(s2, u2, u1), u0);
    const double lg = (double)(e - 1) + fma(sv, h, LG[j]);
    return (int32_t)floor(lg * 8388608.0 + 0.5);
}
__device__ __forceinline__ int32_t lpvip_db(const double *lp, uint32_t d) {
    if (d < 0x800000u) return lpvip_db_near(lp, d);
    uint32_t u = mitchell_exp2_neg(d);
    uint64_t sq = ((uint64_t)u * u) >> 23;
    return -(int32_t)(u + (uint32_t)((sq * 0xB8Au) >> 12));
}

template <>
struct red16<LNSHIP_LPVIP> {
    const double *lp;   // LDS: the db tables (host_tables::lpdb)
    using acc_t = acc_ls;
    __device__ __forceinline__ acc_t start(uint32_t v, uint32_t &) const {
        return {(v & k16_logmask) << 16, (v & k16_sign) << 16};
    }
    // lpvip_sb and lpvip_db formed side by side, without branches, but for
    // the FP64 Gaussian log (opposite signs below one binade), which only
    // lanes that need it run; exact cancellation (d = 0, opposite signs)
    // gives +0
    __device__ __forceinline__ void add_ls(acc_t &a, uint32_t tl16, uint32_t ts16, uint32_t &) const {
        const uint32_t tl = tl16 << 16, ts = ts16 << 16;
        const uint32_t mx = max(a.l, tl), d = mx - min(a.l, tl);
        const uint32_t sgn = a.l > tl ? a.s : ts;
        const bool usedb = (a.s ^ ts) != 0;
        // Mitchell's antilog of -d (0 from 31 binades on), then sb's and db's
        // corrections of it, all products of 24-bit operands (u <= 2^23):
        // u (2^23 - u) >> 23 < 2^21, so its product with 0x2B8 fits 32 bits;
        // u^2 >> 23 <= 2^23, its product with 0xB8A taken as 48 bits
        const uint32_t u = ((0x1000000u - (d & 0x7fffffu)) >> 1) >> min(d >> 23, 31u);
        const uint32_t pc = (uint32_t)(((uint64_t)u * (uint64_t)(0x800000u - u)) >> 23);
        const uint32_t pq = (uint32_t)(((uint64_t)u * u) >> 23);
        const int32_t sb = (int32_t)(u + (mul_u24(pc, 0x2B8u) >> 11));
        const int32_t dbm = -(int32_t)(u + __builtin_amdgcn_alignbit(mulhi_u24(pq, 0xB8Au), mul_u24(pq, 0xB8Au), 12));
        int32_t adj = usedb ? dbm : sb;
        if (usedb && d - 1u < 0x7fffffu) adj = lpvip_db_near(lp, d);
        adj = d < k32_esszer ? adj : 0;
        const uint32_t s = mx + (uint32_t)adj;
        const uint32_t l = (s & k32_sign) ? ((s & k32_one) ? 0u : k32_logmask) : s;
        const bool cancel = d == 0 && usedb;
        a.l = cancel ? 0u : l;
        a.s = cancel ? 0u : sgn;
    }
    __device__ __forceinline__ void add(acc_t &a, uint32_t v, uint32_t &st) const { add_ls(a, v & k16_logmask, v & k16_sign, st); }
    // add() of a positive v to a positive sum: sb only, the sign stays +
    __device__ __forceinline__ void add_pos(acc_t &a, uint32_t v, uint32_t &) const {
        const uint32_t tl = (v & k16_logmask) << 16;
        const uint32_t mx = max(a.l, tl), d = mx - min(a.l, tl);
        const uint32_t u = ((0x1000000u - (d & 0x7fffffu)) >> 1) >> min(d >> 23, 31u);
        const uint32_t pc = (uint32_t)(((uint64_t)u * (uint64_t)(0x800000u - u)) >> 23);
        const int32_t adj = d < k32_esszer ? (int32_t)(u + (mul_u24(pc, 0x2B8u) >> 11)) : 0;
        const uint32_t s = mx + (uint32_t)adj;
        a.l = (s & k32_sign) ? ((s & k32_one) ? 0u : k32_logmask) : s;
    }
    __device__ __forceinline__ uint32_t finish(const acc_t &a) const { return (a.s | a.l) >> 16; }
};

// Stages the tables a reduction needs into LDS (with the sentinels); returns
// the policy.
// Copies n > 0 int4 from global memory to LDS.  Each thread issues its loads
// in batches of B before the first store of the batch, so a batch costs one
// memory round trip instead of B (a launch of a chain kernel stages its
// tables before the chain can start, and the chain waits for every byte).
// Past the end a thread copies the last element again, to the same place and
// with the same value: the batch has no branch for the compiler to sink a
// load into, so the loads issue back to back.
template <int B = 16>
__device__ __forceinline__ void stage_copy(int4 *dst, const int4 *__restrict__ src, int n) {
    for (int i0 = threadIdx.x; i0 < n; i0 += B * (int)blockDim.x) {
        int4 r[B];
#pragma unroll
        for (int j = 0; j < B; j++) r[j] = src[min(i0 + j * (int)blockDim.x, n - 1)];
#pragma unroll
        for (int j = 0; j < B; j++) dst[min(i0 + j * (int)blockDim.x, n - 1)] = r[j];
    }
}

template <int MODE>
__device__ __forceinline__ red16<MODE> stage_tables(const dev_tables &T, char *lds);

template <>
__device__ __forceinline__ red16<LNSHIP_BASE> stage_tables<LNSHIP_BASE>(const dev_tables &T, char *lds) {
    int16_t *g = reinterpret_cast<int16_t *>(lds);
    for (int i = threadIdx.x; i < k16_gauss_n; i += blockDim.x) {
        g[2 * i] = T.gauss16[i];
        g[2 * i + 1] = i == 0 ? (int16_t)-32768 : T.gauss16[k16_gauss_n + i];
    }
    return red16<LNSHIP_BASE>{lds};
}
template <>
__device__ __forceinline__ red16<LNSHIP_MONTE> stage_tables<LNSHIP_MONTE>(const dev_tables &T, char *lds) {
    int32_t *g = reinterpret_cast<int32_t *>(lds);
    stage_copy<8>(reinterpret_cast<int4 *>(g), reinterpret_cast<const int4 *>(T.gauss16m), k16_mc_n);
    // db at distance 0: an adjustment that clamps the log to 0 (exact
    // cancellation; the sign is cleared by the caller).  Thread 0 copied
    // that entry itself, so its own later store wins.
    if (threadIdx.x == 0) g[2] = -(1 << 30);
    return red16<LNSHIP_MONTE>{g, lds_addr(g)};
}
// img: one of the two images built at init (lds32_image): the multi-chain
// step's, or the single-chain step's
__device__ __forceinline__ red16<LNSHIP_SUM32> stage_x32(const int32_t *img, char *lds) {
    int32_t *t = reinterpret_cast<int32_t *>(lds);
    // one copy, in one batch of loads per thread at 256 threads
    stage_copy<32>(reinterpret_cast<int4 *>(t + kl_dlo), reinterpret_cast<const int4 *>(img), (kl_end - kl_dlo) / 4);
    // descriptor of key = (opposite signs) << 8 | (d >> 23): (origin, grid
    // shift, cap of e, lane mask).  Direct keys read the interpolation at d:
    // the sb / db table of d's binade, or the zero pair with a shift that
    // empties d >> sh from the essential zero on; their cap 0 clamps e to 0
    // (and the addend outside the interpolation to 0).  Cotransformation keys
    // (opposite signs, d below two binades) read at e instead: sb's near
    // grid, the far one chosen from e, a cap at the exact-cancellation node
    // (no e reaches past it), and an all-ones mask.
    {
        const uint32_t tb = lds_addr(t), zero = tb + (uint32_t)kl_zero * 4;
        for (int k = threadIdx.x; k < k32_desc_n; k += blockDim.x) {
            const uint32_t q = (uint32_t)k & 255u;
            uint32_t base = zero, sh = 31, cap = 0, co = 0;
            if (k < 256) {
                if (q < (k32_sb_end >> 23)) base = tb + kb_sb, sh = k32_sb_sh;
                else if (q < (k32_esszer >> 23)) base = tb + kb_sbf, sh = k32_sb_fsh;
            } else if (q < (k32_co_end >> 23)) {
                base = tb + kb_sb, sh = k32_sb_sh, cap = k32_co_cancel, co = ~0u;
            } else if (q < (k32_db_end >> 23)) {
                base = tb + kb_db, sh = k32_db_sh;
            } else if (q < (k32_esszer >> 23)) {
                base = tb + kb_dbf, sh = k32_db_fsh;
            }
            // opposite-sign direct keys index with du = d + 2^31
            if (k >= 256 && co == 0) base -= (0x80000000u >> sh) << 2;
            t[kl_desc + 4 * k] = (int32_t)base;
            t[kl_desc + 4 * k + 1] = (int32_t)sh;
            t[kl_desc + 4 * k + 2] = (int32_t)cap;
            t[kl_desc + 4 * k + 3] = (int32_t)co;
        }
    }
    return red16<LNSHIP_SUM32>{x32_origins(t)};
}
template <>
__device__ __forceinline__ red16<LNSHIP_SUM32> stage_tables<LNSHIP_SUM32>(const dev_tables &T, char *lds) {
    return stage_x32(T.lds32, lds);
}
template <>
__device__ __forceinline__ red16<LNSHIP_LPVIP> stage_tables<LNSHIP_LPVIP>(const dev_tables &T, char *lds) {
    stage_copy<4>(reinterpret_cast<int4 *>(lds), reinterpret_cast<const int4 *>(T.lpdb), 3 * k_lp_n * 8 / 16);
    return red16<LNSHIP_LPVIP>{reinterpret_cast<const double *>(lds)};
}
// the pair image of the positive-sum adder
__device__ __forceinline__ pos_tab stage_pos32(const dev_tables &T, char *lds) {
    stage_copy<32>(reinterpret_cast<int4 *>(lds), reinterpret_cast<const int4 *>(T.pos32), k_lds_pos32 / 16);
    uint32_t tb = lds_addr(lds);
    asm("" : "+v"(tb));
    pos_tab P{tb, tb + (uint32_t)(kp32_near - (int)(k32_sb_end >> k32_sb_fsh)) * 8u, 1u, 0u};
    asm("" : "+v"(P.near), "+v"(P.far), "+v"(P.one), "+v"(P.zero));
    return P;
}
// the tables of a kernel whose xlns32 additions are single-chain steps
// (x32_add_step) when DEC, else multi-chain ones (x32_add_ls)
template <int MODE, bool DEC>
__device__ __forceinline__ red16<MODE> stage_for(const dev_tables &T, char *lds) {
    if constexpr (MODE == LNSHIP_SUM32 && DEC) return stage_x32(T.lds32d, lds);
    else return stage_tables<MODE>(T, lds);
}

template <int MODE>
constexpr int lds_tables_bytes() {
    return MODE == LNSHIP_BASE ? 2 * k16_gauss_n * 2 :
           MODE == LNSHIP_MONTE ? 4 * k16_mc_n * 4 :
           MODE == LNSHIP_SUM32 ? k_lds_tab32 : 3 * k_lp_n * 8;
}
// The LDS tables of the xlns16 row kernels (rms_norm, soft_max): their sum32
// chains add only positive values (squares, exps), over the positive-sum
// adder's pair image; the other modes stage their adder's tables.
template <int MODE>
constexpr int row_tables_bytes() {
    return MODE == LNSHIP_SUM32 ? k_lds_pos32 : lds_tables_bytes<MODE>();
}
template <int MODE>
__device__ __forceinline__ red16<MODE> stage_rows(const dev_tables &T, char *lds, pos_tab &P) {
    if constexpr (MODE == LNSHIP_SUM32) {
        P = stage_pos32(T, lds);
        return red16<MODE>{};
    } else {
        return stage_tables<MODE>(T, lds);
    }
}

// ---- MUL_MAT ------------------------------------------------------------------
// One lane per weight row m and NC activation columns n (NC independent
// accumulations interleaved for latency hiding).  With XL the workgroup first
// converts its NC activation rows into LDS (F32 -> xlns16 through the
// conversion table) and lanes read them back with wave-uniform 16-byte LDS
// reads; without XL (rows too long for LDS) k_act has converted them into xs
// [slice][N][Kp] and they come from global memory through vector loads.  A
// wave-uniform global load would otherwise become a scalar load, and since
// scalar loads and LDS reads share one completion counter (and scalar loads
// return out of order) every table read would then also wait for it.  The
// weights (and activations) of the next PF groups of eight k are in flight
// while a group is accumulated.

struct mm_args16 {
    const uint16_t *w;
    const uint16_t *x;    // converted activations [slice][N][Kp] (without XL)
    const float *xf;      // F32 activations (XL): row n of slice z at z * x_slice + n * x_ld
    float *dst;
    int64_t K, kp, M, N;
    int64_t x_ld, x_slice;
    int64_t ne02, ne12, r2, r3;
    int64_t w_mstride, w_slice, dst_ld, dst_slice;
    uint32_t seed;
    const uint16_t *state;   // Monte start read on the device (null: seed)
    uint64_t offset;
    // MUL_MAT_ID (ids non-null): slice z = (slot i12, token i13) multiplies
    // expert ids[i12 + i13 ids_t] (of n_w) by activation slice
    // i13 x_bcast + i12 % x_bcast; an expert out of range skips the slice
    // and is recorded in err
    const int32_t *ids;
    int64_t ids_t, x_bcast, n_w;
    unsigned long long *err;
    const float *resid;   // non-null: dst = resid + W x (the graph's ADD), resid laid out as dst
    // k_mm16_rms: x = rms_norm(xf) * norm (norm: K floats), epsilon eps; skew
    // is added to the predicted scale code (0; a test hook sets it)
    const float *norm;
    float eps;
    uint32_t skew;
    uint32_t rms_ik, rms_eps;   // the xlns16 codes of 1 / K and of eps (from the host's table)
    // non-null (XL launches): the activation is swiglu(xf, glu_up), the GLU
    // node before the mul_mat: up row n at glu_up + n * x_ld
    const float *glu_up;
    // k_mm16 with norm (XL launches of one slice): the RMS_NORM node's
    // Monte start, monte_start(rms_seed, state, rms_offset)
    uint32_t rms_seed;
    uint64_t rms_offset;
    // set by the launcher: the grid is 2^xcd_sh times wider than the work;
    // workgroup x works (as block x >> xcd_sh) iff x is a multiple of 2^xcd_sh
    uint32_t xcd_sh;
};

// Records an index out of range: err[0] = 1, err[1] = the first such index.
__device__ __forceinline__ void index_fault(unsigned long long *err, int64_t idx) {
    if (atomicCAS(&err[0], 0ull, 1ull) == 0ull) err[1] = (unsigned long long)idx;
}

// The weight slice and activation slice of grid slice (i12, i13): ggml's
// broadcast for MUL_MAT, the expert of the slot for MUL_MAT_ID.  Returns
// false when the expert is out of range.
template <class A>
__device__ __forceinline__ bool mm_slices(const A &a, int64_t z, int64_t i12, int64_t i13, int64_t &zw, int64_t &zx) {
    if (!a.ids) {
        zw = (i13 / a.r3) * a.ne02 + i12 / a.r2;
        zx = z;
        return true;
    }
    zx = i13 * a.x_bcast + i12 % a.x_bcast;
    zw = a.ids[i12 + i13 * a.ids_t];
    if (zw >= 0 && zw < a.n_w) return true;
    index_fault(a.err, zw);
    return false;
}

// A Monte op's starting LFSR state: the seed, or a jump from a state read on
// the device when the op runs.
__device__ __forceinline__ uint32_t monte_start(const dev_tables &T, uint32_t seed, const uint16_t *state,
                                                uint64_t offset) {
    return state ? lfsr_jump(T, *state, offset) : seed;
}

template <int MODE>
constexpr int mm_xl_offset() { return (lds_tables_bytes<MODE>() + 15) & ~15; }
// LDS padding past the activation rows (a block's prefetch reads up to that
// far past the last column)
constexpr int k_xl_pad = 8 * 16;

__device__ __forceinline__ uint32_t half16(uint32_t w, int hi) { return hi ? (w >> 16) : (w & 0xffffu); }

// The first weights of lane m's chains (group 0, then the block of groups
// 1 .. PF), as mm16_chains loads them.  A decode GEMV loads them before it
// stages its tables, so that their HBM latency passes meanwhile.
template <int PF>
struct mm_head {
    uint4 w0, w[PF];
};
// the weights of groups g0 .. g0 + PF - 1 of lane m in weight slice zw (past
// the slice's last group: the last group again)
template <int PF>
__device__ __forceinline__ void mm16_wblock(const mm_args16 &a, int64_t m, int64_t zw, int g0, uint4 (&w)[PF]) {
    // from the block's first group (a wave-uniform base, clamped to the
    // slice's last group) at lane offset m * 16 plus p * (bytes between
    // groups) for the block's group p, the offset capped at the last group's
    const int last = (int)(a.kp >> 3) - 1;
    const char *wsl = reinterpret_cast<const char *>(a.w + zw * a.w_slice);
    const uint64_t gsb = (uint64_t)a.w_mstride * 16;
    const int gb = min(g0, last);
    const char *wb = wsl + (uint64_t)gb * gsb;
    const uint32_t cap = (uint32_t)((uint64_t)(last - gb) * gsb) + (uint32_t)m * 16;
#pragma unroll
    for (int p = 0; p < PF; p++)
        w[p] = *reinterpret_cast<const uint4 *>(wb + min((uint32_t)((uint64_t)m * 16 + (uint64_t)p * gsb), cap));
}
template <int PF>
__device__ __forceinline__ mm_head<PF> mm16_head(const mm_args16 &a, int64_t m, int64_t zw) {
    mm_head<PF> h;
    h.w0 = *reinterpret_cast<const uint4 *>(a.w + zw * a.w_slice + m * 8);
    mm16_wblock<PF>(a, m, zw, 1, h.w);
    return h;
}

// The K-long chains of lane m (output row m of slice z) over columns
// n0 .. n0 + nc: the weights from HBM, the activations from the LDS rows at
// xl (XL) or the converted rows in scratch; each column's finished
// accumulator (an xlns16 code) into res.  HEAD: the first weights come
// loaded in head.
template <int MODE, int NC, int PF, bool XL, bool HEAD = false>
__device__ __forceinline__ void mm16_chains(const mm_args16 &a, const dev_tables &T, const red16<MODE> &R,
                                            const uint16_t *xl, int64_t m, int64_t z, int64_t zw, int64_t zx,
                                            int64_t n0, int nc, uint32_t (&res)[NC],
                                            const mm_head<PF> &head = mm_head<PF>{}) {
    const int kp = (int)a.kp;
    const uint16_t *ws = a.w + zw * a.w_slice + m * 8;
    const uint16_t *xs = a.x + (zx * a.N + n0) * a.kp;
    const int64_t wstride = a.w_mstride * 8;   // between consecutive groups of 8 k
    typename red16<MODE>::acc_t acc[NC]{};
    uint32_t st[NC];
#pragma unroll
    for (int j = 0; j < NC; j++) {
        st[j] = 0;
        if (MODE == LNSHIP_MONTE && j < nc) {
            const uint64_t out = ((uint64_t)z * (uint64_t)a.M + (uint64_t)m) * (uint64_t)a.N + (uint64_t)(n0 + j);
            st[j] = lfsr_jump(T, monte_start(T, a.seed, a.state, a.offset), out * (uint64_t)(a.K - 1));
        }
    }
    const int K = (int)a.K;
    const int full = K >> 3, tail = K & 7;
    // Prefetches past the last group reload the last group: every load is
    // unconditional, so the compiler can count outstanding loads exactly and
    // wait only for the one a step needs.
    const int last = (kp >> 3) - 1;
    auto load_w = [&](int g) { return *reinterpret_cast<const uint4 *>(ws + (int64_t)min(g, last) * wstride); };
    auto load_x = [&](int j, int g) {
        // the offset goes through a vector register: the value then counts as
        // per-lane, so a global read is a vector load (not a scalar one) and an
        // LDS read is waited for where it is used, not copied to scalar
        // registers as soon as it is issued
        int64_t off = (int64_t)(XL || j < nc ? j : 0) * kp + (int64_t)min(g, last) * 8;
        asm("" : "+v"(off));
        return *reinterpret_cast<const uint4 *>((XL ? xl : xs) + off);
    };
    // steps [u0, u1) of a group: the product (xlns16_mul: log fields added
    // and clamped, signs xor'ed), then one reduction step per column
    // SUM32, one chain per lane: what the chain carries from group to group
    // (the product of the next step, its opposite-signs flag, and the
    // product pair of the next group's steps 0 and 1)
    uint32_t c_tl = 0, c_ts = 0, c_uf = 0, c_pl = 0, c_ps = 0;
    // masks in registers (short encodings of the instructions that take them)
    uint32_t k_lm = 0x7fff7fffu, k_sg = k32_sign, k_hi = 0xffff0000u;
    asm("" : "+v"(k_lm), "+v"(k_sg), "+v"(k_hi));
    // steps [u0, u1) of a group; wn / xn: the next group's data.  fresh: the
    // chain's first group, or one whose carried state was not formed from it
    auto steps = [&](const uint4 &wq, const uint4 (&xq)[NC], const uint4 &wn, const uint4 (&xn)[NC], int u0, int u1,
                     bool fresh) {
        const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w};
        if constexpr (MODE == LNSHIP_SUM32 && NC == 1) {
            const uint32_t xx[4] = {xq[0].x, xq[0].y, xq[0].z, xq[0].w};
            // the products of steps 2i and 2i + 1 together, in the two 16-bit
            // halves: the log fields added (no carry crosses the halves: each
            // sum is at most 0x7fff + 0x7fff), less the offset with unsigned
            // saturation (underflow: log 0), capped at 0x7fff (overflow); and
            // the sign bits xor'ed.  Pair i + 1 is formed in step 2i's second
            // round trip, the next group's pair 0 in step 6's.
            uint32_t pl[4], ps[4];
            auto pair = [&](uint32_t w, uint32_t x, uint32_t &l, uint32_t &sg) {
                const uint32_t lm = (w & k_lm) + (x & k_lm);
                l = pk_min_u16(pk_sub_sat_u16(lm, 0x40004000u), 0x7fff7fffu);
                sg = w ^ x;
            };
            // the product of step u (xlns32 positions) from its pair
            auto half = [&](int u, uint32_t l, uint32_t sg, uint32_t &tl, uint32_t &ts) {
                if ((u & 1) == 0) {
                    tl = l << 16;
                    ts = (sg << 16) & k_sg;
                } else {
                    tl = l & k_hi;
                    ts = sg & k_sg;
                }
            };
            // u0 is 0, or -1 for the chain's first group (its step 0 starts
            // the sum)
            const bool first = u0 < 0;
            const int ub = 0;
            if (fresh) {
                pair(ww[0], xx[0], pl[0], ps[0]);
                half(ub, pl[0], ps[0], c_tl, c_ts);
                c_uf = acc[0].s ^ c_ts;
            } else {
                pl[0] = c_pl;
                ps[0] = c_ps;
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (u >= ub && u < u1) {
                    uint32_t ntl = 0, nts = 0;
                    // the next step's product, from its pair (after step 7,
                    // the next group's step 0 from the carried pair): its
                    // sign in this step's first round trip, its log in the
                    // second
                    auto next = [&] {
                        uint32_t l_unused;
                        if (u + 1 < u1) half(u + 1, pl[(u + 1) >> 1], ps[(u + 1) >> 1], l_unused, nts);
                        else if (u == 7) half(0, c_pl, c_ps, l_unused, nts);
                        return nts;
                    };
                    auto post = [&] {
                        uint32_t s_unused;
                        if ((u & 1) == 0 && u < 6) pair(ww[(u >> 1) + 1], xx[(u >> 1) + 1], pl[(u >> 1) + 1], ps[(u >> 1) + 1]);
                        if (u + 1 < u1) half(u + 1, pl[(u + 1) >> 1], ps[(u + 1) >> 1], ntl, s_unused);
                        else if (u == 7) half(0, c_pl, c_ps, ntl, s_unused);
                        if (u == 6) pair(wn.x, xn[0].x, c_pl, c_ps);
                    };
                    if (first && u == 0) {
                        acc[0] = {c_tl, c_ts};
                        c_uf = c_ts ^ next();
                        post();
                    } else {
                        c_uf = x32_add_step(R.O, acc[0], c_tl, c_ts, c_uf, next, post);
                    }
                    c_tl = ntl;
                    c_ts = nts;
                }
            }
            return;
        }
        if constexpr (MODE == LNSHIP_SUM32) {
            // several chains per lane: the products of steps 2i and 2i + 1 of
            // a chain together, in the two 16-bit halves (as in the single
            // chain above).  The weights' logs, shared by the chains, less the
            // offset once (wl - 0x4000 in [-0x4000, 0x3fff] as int16); then
            // per chain wl - 0x4000 + xl, saturated at 0x7fff by the signed
            // add and at 0 by the maximum: the clamped product log
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (2 * i + 1 < u0 || 2 * i >= u1) continue;
                const uint32_t wb = pk_sub_u16(ww[i] & k_lm, 0x40004000u);
#pragma unroll
                for (int j = 0; j < NC; j++) {
                    const uint32_t xv = i == 0 ? xq[j].x : i == 1 ? xq[j].y : i == 2 ? xq[j].z : xq[j].w;
                    const uint32_t pl = pk_add_sat_nonneg_i16(wb, xv & k_lm);
                    const uint32_t ps = ww[i] ^ xv;
#pragma unroll
                    for (int h = 0; h < 2; h++) {
                        const int u = 2 * i + h;
                        if (u < u0 || u >= u1) continue;
                        const uint32_t tl = h == 0 ? pl << 16 : pl & k_hi;
                        const uint32_t ts = h == 0 ? (ps << 16) & k_sg : ps & k_sg;
                        if (u == 0 && u0 < 0) acc[j] = {tl, ts};
                        else x32_add_ls(R.O, acc[j], tl, ts);
                    }
                }
            }
            return;
        }
        if constexpr (NC == 1) {
            // one chain: the products of steps 2i and 2i + 1 together in the
            // two 16-bit halves (as the sum32 chain forms them), then each
            // step's log and sign from its half
            const uint32_t xx[4] = {xq[0].x, xq[0].y, xq[0].z, xq[0].w};
            uint32_t pl[4], ps[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                if (2 * i + 1 < u0 || 2 * i >= u1) continue;
                pl[i] = pk_min_u16(pk_sub_sat_u16((ww[i] & k_lm) + (xx[i] & k_lm), 0x40004000u), 0x7fff7fffu);
                ps[i] = ww[i] ^ xx[i];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (u >= u0 && u < u1) {
                    const uint32_t tl = (u & 1) ? pl[u >> 1] >> 16 : pl[u >> 1] & 0xffffu;
                    const uint32_t ts = ((u & 1) ? ps[u >> 1] >> 16 : ps[u >> 1]) & k16_sign;
                    if (u == 0 && u0 < 0) acc[0] = R.start(ts | tl, st[0]);
                    else R.add_ls(acc[0], tl, ts, st[0]);
                }
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (u >= u0 && u < u1) {
                const uint32_t wv = half16(ww[u >> 1], u & 1);
                const uint32_t wl = wv & k16_logmask;
#pragma unroll
                for (int j = 0; j < NC; j++) {
                    const uint32_t xv = half16(u < 2 ? xq[j].x : u < 4 ? xq[j].y : u < 6 ? xq[j].z : xq[j].w, u & 1);
                    const int32_t l = (int32_t)wl + (int32_t)(xv & k16_logmask) - (int32_t)k16_one;
                    const uint32_t tl = (uint32_t)min(max(l, 0), (int32_t)k16_logmask);
                    const uint32_t ts = (wv ^ xv) & k16_sign;
                    if (u == 0 && u0 < 0) acc[j] = R.start(ts | tl, st[j]);
                    else R.add_ls(acc[j], tl, ts, st[j]);
                }
            }
        }
    };
    {
        // group 0 starts the accumulation (u0 = -1 marks the start step)
        uint4 xq[NC];
#pragma unroll
        for (int j = 0; j < NC; j++) xq[j] = load_x(j, 0);
        const uint4 wq = HEAD ? head.w0 : load_w(0);
        // groups 1 .. full-1 in blocks of PF, double-buffered: the loads of
        // block b + 1 are issued together before block b is accumulated
        uint4 wa[PF], wb[PF], xa[PF][NC], xb[PF][NC];
        // A block's loads from bases that move once per block: the weights
        // as mm16_wblock (the last block's prefetch past the slice rereads
        // the last group); activations in LDS at immediate offsets p * 16
        // from the block's base (the LDS copy has PF * 16 bytes of padding
        // past its last column).
        auto load_xblock = [&](uint4 (&x)[PF][NC], int g0) {
#pragma unroll
            for (int j = 0; j < NC; j++) {
                if constexpr (XL) {
                    // the base through a vector register: the data then counts
                    // as per-lane and is waited for where it is used
                    int32_t xo = (j * kp + g0 * 8) * 2;
                    asm("" : "+v"(xo));
                    const char *xb = reinterpret_cast<const char *>(xl) + xo;
#pragma unroll
                    for (int p = 0; p < PF; p++) x[p][j] = *reinterpret_cast<const uint4 *>(xb + p * 16);
                } else {
#pragma unroll
                    for (int p = 0; p < PF; p++) x[p][j] = load_x(j, g0 + p);
                }
            }
        };
        auto load_block = [&](uint4 (&w)[PF], uint4 (&x)[PF][NC], int g0) {
            mm16_wblock<PF>(a, m, zw, g0, w);
            load_xblock(x, g0);
        };
        // the next group of group p of a block is p + 1, or the first of the
        // other buffer (loaded before this block runs)
        auto run_block = [&](const uint4 (&w)[PF], const uint4 (&x)[PF][NC], const uint4 (&wo)[PF],
                             const uint4 (&xo)[PF][NC], int g0) {
#pragma unroll
            for (int p = 0; p < PF; p++)
                if (g0 + p < full) steps(w[p], x[p], p + 1 < PF ? w[p + 1] : wo[0], p + 1 < PF ? x[p + 1] : xo[0], 0, 8, false);
        };
        if constexpr (HEAD) {
#pragma unroll
            for (int p = 0; p < PF; p++) wa[p] = head.w[p];
            load_xblock(xa, 1);
        } else {
            load_block(wa, xa, 1);
        }
        steps(wq, xq, wa[0], xa[0], -1, full > 0 ? 8 : tail, true);
        for (int g = 1; g < full; g += 2 * PF) {
            load_block(wb, xb, g + PF);
            run_block(wa, xa, wb, xb, g);
            if (g + PF >= full) break;
            load_block(wa, xa, g + 2 * PF);
            run_block(wb, xb, wa, xa, g + PF);
        }
        if (full > 0 && tail > 0) {
            uint4 tx[NC];
#pragma unroll
            for (int j = 0; j < NC; j++) tx[j] = load_x(j, full);
            const uint4 tw = load_w(full);
            steps(tw, tx, tw, tx, 0, tail, true);
        }
    }
#pragma unroll
    for (int j = 0; j < NC; j++) res[j] = R.finish(acc[j]) & 0xffffu;
}

// W < 64: W rows per wave (single-chain GEMVs, bound by the dependent
// latency of their chains).  sum32: the wave's other lanes only stage the
// tables and the activations (a VALU instruction with only the first 16
// lanes active completes sooner, and the step with it).  The other modes run
// each row's chain on 64 / W lanes, so that every lane stays active: their
// steps branch (lpvip's FP64 Gaussian log, the sign cases) and, measured,
// run slower with part of the wave inactive (lpvip K 1536: 420 us with 16
// lanes, 334 us with the same 16 chains on all 64, 313 us with 4 chains)
template <int MODE, int NC, int PF, bool XL, int CG, int W = 64>
__global__ __launch_bounds__(k_block * CG) void k_mm16(mm_args16 a, dev_tables T) {
    extern __shared__ __align__(16) char lds[];
    // a widened launch: the workgroups between the working ones leave at once
    if (blockIdx.x & ((1u << a.xcd_sh) - 1u)) return;
    // CG column groups of k_block lanes each share the staged tables: group
    // c takes columns [nw + c NC, nw + (c + 1) NC) of the same k_block rows
    const int cg = CG == 1 ? 0 : (int)(threadIdx.x / k_block);
    const int64_t nw = (int64_t)blockIdx.y * (NC * CG);
    const int64_t n0 = nw + (int64_t)cg * NC;
    const int64_t z = blockIdx.z;
    const int64_t i12 = z % a.ne12, i13 = z / a.ne12;
    const int ncw = (int)min<int64_t>(NC * CG, a.N - nw);
    const int nc = (int)max<int64_t>(0, min<int64_t>(NC, a.N - n0));
    const int kp = (int)a.kp;
    int64_t zw, zx;
    const bool slice_ok = mm_slices(a, z, i12, i13, zw, zx);
    const int lane = (int)(threadIdx.x & 63u);
    constexpr bool dup = W < 64 && MODE != LNSHIP_SUM32;   // a chain on 64 / W lanes
    const int wr = dup ? lane / (64 / W) : lane;              // the lane's row in the wave
    const int64_t m = W < 64 ? (int64_t)(blockIdx.x >> a.xcd_sh) * (k_block / 64 * W) + (threadIdx.x >> 6) * W + wr
                             : (int64_t)(blockIdx.x >> a.xcd_sh) * k_block + (threadIdx.x % k_block);
    const bool live = !(W < 64 && !dup && lane >= W) && m < a.M && nc > 0 && slice_ok;
    // one-column launches: the chain's first weights loaded before the
    // tables are staged (their HBM latency passes meanwhile)
    constexpr bool head = NC == 1 && XL;
    mm_head<PF> hw{};
    if (head && live && a.K > 0) hw = mm16_head<PF>(a, m, zw);
    const red16<MODE> R = stage_for<MODE, NC == 1>(T, lds);
    uint16_t *xl = reinterpret_cast<uint16_t *>(lds + mm_xl_offset<MODE>());
    // The RMS_NORM and MUL nodes before the product (norm): each workgroup
    // forms the scales of its own columns' rows, as k_rms16 does: the
    // squares into the activation rows' LDS, then one row's chain per lane
    // of wave 0 (lane l on column l mod ncw, every lane busy); the staging
    // below forms h from them
    __shared__ uint32_t s_rinv[64];
    if (XL && a.norm) {
        const float *xf = a.xf + zx * a.x_slice + nw * a.x_ld;
        const int K = (int)a.K;
        for (int e = threadIdx.x; e < ncw * K; e += k_block * CG) {
            const int j = e / K, k = e - j * K;
            const uint32_t c = x16_from_f32(T.cvt16, xf[(int64_t)j * a.x_ld + k]);
            xl[j * kp + k] = (uint16_t)x16_mul(c, c);
        }
        __syncthreads();
        if (threadIdx.x < 64u) {
            const int j = (int)threadIdx.x % ncw;
            uint32_t s = 0;
            if constexpr (MODE == LNSHIP_MONTE)
                s = lfsr_jump(T, monte_start(T, a.rms_seed, a.state, a.rms_offset), (uint64_t)(nw + j) * (uint64_t)K);
            typename red16<MODE>::acc_t acc = R.start(0u, s);
            chain16<red16<MODE>, true>(R, acc, xl + j * kp, 0, K, s);   // squares: positive
            const uint32_t mean = x16_mul(R.finish(acc) & 0xffffu, a.rms_ik);
            // the epsilon add is a plain xlns16_add in every mode
            if ((int)threadIdx.x < ncw) s_rinv[j] = x16_recip(x16_sqrt(x16_add_g(T.gauss16, mean, a.rms_eps)));
        }
        __syncthreads();
    }
    if (XL) {
        // columns past N and k past K hold xlns16 zero
        // in batches of eight per thread: the loads, then the conversion
        // table's lookups, then the stores (two memory round trips a batch).
        // The staging with the rms_norm's scale is a loop of its own, so the
        // plain and GLU launches keep theirs as they were.
        const float *xf = a.xf + zx * a.x_slice + nw * a.x_ld;
        constexpr int nt = k_block * CG, B = 8;
        const int kl = (int)a.K - 1;
        auto stage = [&](auto norm_tag) __attribute__((always_inline)) {
            constexpr bool NORM = decltype(norm_tag)::value;
            for (int j = 0; j < NC * CG; j++) {
                if (kl < 0) {
                    for (int k = threadIdx.x; k < kp; k += nt) xl[j * kp + k] = 0;
                    continue;
                }
                // loads and lookups stay in the row; only the stores are bounded
                const float *row = xf + (int64_t)min(j, ncw - 1) * a.x_ld;
                const uint32_t inv = NORM ? s_rinv[min(j, ncw - 1)] : 0u;
                for (int k0 = threadIdx.x; k0 < kp; k0 += B * nt) {
                    float v[B];
#pragma unroll
                    for (int q = 0; q < B; q++) v[q] = row[min(k0 + q * nt, kl)];
                    uint32_t c[B];
#pragma unroll
                    for (int q = 0; q < B; q++) c[q] = x16_from_f32(T.cvt16, v[q]);
                    if constexpr (NORM) {
                        // the RMS_NORM node's output, then the MUL node's by
                        // the norm weight, each through F32 (rho16)
                        float g[B];
#pragma unroll
                        for (int q = 0; q < B; q++) g[q] = a.norm[min(k0 + q * nt, kl)];
#pragma unroll
                        for (int q = 0; q < B; q++)
                            c[q] = T.rho16[x16_mul(T.rho16[x16_mul(c[q], inv)], x16_from_f32(T.cvt16, g[q]))];
                    } else if (a.glu_up) {
                        // swiglu as its node computes it (silu(gate) * up in
                        // xlns16, F32 out), then into xlns16 as here
                        const float *urow = a.glu_up + zx * a.x_slice + (nw + (int64_t)min(j, ncw - 1)) * a.x_ld;
                        float u[B];
#pragma unroll
                        for (int q = 0; q < B; q++) u[q] = urow[min(k0 + q * nt, kl)];
#pragma unroll
                        for (int q = 0; q < B; q++)
                            c[q] = T.rho16[x16_mul(x16_mul(c[q], T.sig16[c[q]]), x16_from_f32(T.cvt16, u[q]))];
                    }
                    // every code in a register before the bounded stores: none
                    // of the batch's loads moves into a store's branch
#pragma unroll
                    for (int q = 0; q < B; q++) asm volatile("" ::"v"(c[q]));
#pragma unroll
                    for (int q = 0; q < B; q++) {
                        const int k = k0 + q * nt;
                        if (k < kp) xl[j * kp + k] = (j < ncw && k <= kl) ? (uint16_t)c[q] : (uint16_t)0;
                    }
                }
            }
        };
        if (a.norm) stage(std::true_type{});
        else stage(std::false_type{});
        xl += cg * NC * kp;
    }
    __syncthreads();

    if (!live) return;
    float *ds = a.dst + z * a.dst_slice + n0 * a.dst_ld + m;
    // output j of code c, with the fused ADD of the residual when there is
    // one: the F32 result and the residual through xlns16 (the result's
    // round trip in one lookup, rho16), added, back to F32 (the ADD node's
    // arithmetic)
    auto put = [&](int j, uint32_t c) {
        const int64_t o = (ds - a.dst) + (int64_t)j * a.dst_ld;
        a.dst[o] = a.resid ? T.rev16[x16_add_g(T.gauss16, T.rho16[c], x16_from_f32(T.cvt16, a.resid[o]))]
                           : T.rev16[c];
    };
    if (a.K == 0) {
        if (!dup || lane % (64 / W) == 0)
            for (int j = 0; j < nc; j++) put(j, 0u);
        return;
    }

    uint32_t res[NC];
    mm16_chains<MODE, NC, PF, XL, head>(a, T, R, xl, m, z, zw, zx, n0, nc, res, hw);
    if (dup && lane % (64 / W) != 0) return;   // one lane of a chain stores
#pragma unroll
    for (int j = 0; j < NC; j++)
        if (j < nc) put(j, res[j]);
}

// xlns32 (the LNS32 backend): plain sequential xlns32_add
struct mm_args32 {
    const uint32_t *w;
    const uint32_t *x;
    float *dst;
    int64_t K, kp, M, N;
    int64_t ne02, ne12, r2, r3;
    int64_t w_mstride, w_slice, dst_ld, dst_slice;
    const int32_t *ids;   // MUL_MAT_ID, as in mm_args16
    int64_t ids_t, x_bcast, n_w;
    unsigned long long *err;
    const float *resid;   // as in mm_args16
    uint32_t xcd_sh;      // as in mm_args16
    // XL launches (one column per workgroup): the F32 activations, row n of
    // slice z at xf + z x_slice + n x_ld, converted into LDS by the launch;
    // with norm, x = rms_norm(xf) * norm (epsilon eps) first, with glu_up,
    // x = swiglu(xf, glu_up) (up row n at glu_up + n x_ld)
    const float *xf;
    int64_t x_ld, x_slice;
    const float *norm;
    float eps;
    const float *glu_up;
};

// (defined with the other sequential row sums below)
__device__ __forceinline__ void chain_pos32(const pos_tab &P, uint32_t &l, const uint32_t *row, int i0, int n);

// xlns32_silu: x times the sigmoid of its value, the sigmoid formed in
// double and rounded to float (libm-independent at float precision)
__device__ __forceinline__ uint32_t x32_silu(uint32_t x) {
    const double v = (double)x32_to_f32(x);
    return x32_mul(x, x32_from_f32((float)(1.0 / (1.0 + exp(-v)))));
}

// One lane per weight row m and NC columns, CG column groups per workgroup
// sharing the staged tables (as k_mm16).  A group of eight k is two 16-byte
// loads of weights and two per column of activations; the next PF groups are
// in flight while one is accumulated.
// W: rows per wave (64, or 16 with the other lanes only staging, as in k_mm16)
// XL: the activation row converted into LDS after the tables by the launch
// (one column per workgroup), its nodes before the product with it (the
// rms_norm and norm MUL, or the swiglu), exactly as they run apart: F32
// between the nodes, each converted as the next node converts it
template <int NC, int PF, int CG, int W = 64, bool XL = false>
__global__ __launch_bounds__(k_block * CG) void k_mm32(mm_args32 a, dev_tables T) {
    static_assert(!XL || (NC == 1 && CG == 1), "XL launches take one column per workgroup");
    extern __shared__ __align__(16) char lds[];
    if (blockIdx.x & ((1u << a.xcd_sh) - 1u)) return;   // as in k_mm16
    uint32_t *xl = reinterpret_cast<uint32_t *>(lds + k_lds_tab32);   // XL: the activation row's codes
    __shared__ uint32_t s_inv;
    int64_t zwx = 0, zxx = 0;
    if constexpr (XL) {
        const int64_t zz = blockIdx.z;
        mm_slices(a, zz, zz % a.ne12, zz / a.ne12, zwx, zxx);
        if (a.norm) {
            // the rms_norm node's sum of squares exactly as k_rms32 forms it:
            // the positive-sum image staged first (where the GEMV's image
            // goes next), the squares into the row's LDS past both images,
            // one chain (every lane of wave 0 runs it)
            const pos_tab P = stage_pos32(T, lds);
            const float *row = a.xf + zxx * a.x_slice + (int64_t)blockIdx.y * a.x_ld;
            const int K = (int)a.K;
            for (int k = threadIdx.x; k < K; k += blockDim.x) {
                const uint32_t c = x32_from_f32(row[k]);
                xl[k] = x32_mul(c, c);
            }
            __syncthreads();
            if (threadIdx.x < 64u) {
                uint32_t acc = 0u;
                chain_pos32(P, acc, xl, 0, K);   // squares: positive
                const uint32_t mean = x32_mul(acc, x32_from_f32(1.0f / (float)K));
                // mean >= 0: the epsilon add is a positive one unless eps < 0
                const uint32_t e = x32_from_f32(a.eps);
                const uint32_t me = (e & k32_sign) ? x32_add(T.tab32, mean, e) : x32_add_pos2(P, mean, e);
                if (threadIdx.x == 0) s_inv = x32_recip(x32_sqrt(me));
            }
            __syncthreads();
        }
    }
    const red16<LNSHIP_SUM32> R = stage_for<LNSHIP_SUM32, NC == 1>(T, lds);
    if constexpr (XL) {
        const float *row = a.xf + zxx * a.x_slice + (int64_t)blockIdx.y * a.x_ld;
        const int K = (int)a.K, kp = (int)a.kp;
        const uint32_t inv = a.norm ? s_inv : 0u;
        const float *urow = a.glu_up ? a.glu_up + zxx * a.x_slice + (int64_t)blockIdx.y * a.x_ld : nullptr;
        for (int k = threadIdx.x; k < kp; k += blockDim.x) {
            uint32_t c = 0u;
            if (k < K) {
                const float f = row[k];
                if (a.norm) {
                    const float y = x32_to_f32(x32_mul(x32_from_f32(f), inv));
                    c = x32_from_f32(x32_to_f32(x32_mul(x32_from_f32(y), x32_from_f32(a.norm[k]))));
                } else if (urow) {
                    c = x32_from_f32(x32_to_f32(x32_mul(x32_silu(x32_from_f32(f)), x32_from_f32(urow[k]))));
                } else {
                    c = x32_from_f32(f);
                }
            }
            xl[k] = c;
        }
    }
    __syncthreads();
    const int cg = CG == 1 ? 0 : (int)(threadIdx.x / k_block);
    const int lane = (int)(threadIdx.x & 63u);
    const int64_t m = W < 64 ? (int64_t)(blockIdx.x >> a.xcd_sh) * (k_block / 64 * W) + (threadIdx.x >> 6) * W + lane
                             : (int64_t)(blockIdx.x >> a.xcd_sh) * k_block + (threadIdx.x % k_block);
    const int64_t n0 = ((int64_t)blockIdx.y * CG + cg) * NC;
    if ((W < 64 && lane >= W) || m >= a.M || n0 >= a.N) return;
    const int64_t z = blockIdx.z;
    const int64_t i12 = z % a.ne12, i13 = z / a.ne12;
    const int nc = (int)min<int64_t>(NC, a.N - n0);
    int64_t zw, zx;
    if (!mm_slices(a, z, i12, i13, zw, zx)) return;
    const uint32_t *ws = a.w + zw * a.w_slice + m * 8;
    const uint32_t *xs = XL ? nullptr : a.x + (zx * a.N + n0) * a.kp;
    const int64_t wstride = a.w_mstride * 8;
    float *ds = a.dst + z * a.dst_slice + n0 * a.dst_ld + m;
    // output j, with the fused ADD of the residual (xlns32 add of the two
    // values, as the ADD node computes it) when there is one
    auto put = [&](int j, float y) {
        const int64_t o = (ds - a.dst) + (int64_t)j * a.dst_ld;
        if (a.resid) y = x32_to_f32(x32_add(T.tab32, x32_from_f32(y), x32_from_f32(a.resid[o])));
        a.dst[o] = y;
    };
    if (a.K == 0) {
        for (int j = 0; j < nc; j++) put(j, 0.0f);
        return;
    }
    struct grp {
        uint4 lo, hi;
    };
    const int K = (int)a.K;
    const int full = K >> 3, tail = K & 7;
    const int last = (int)(a.kp >> 3) - 1;   // loads past the end reload the last group
    auto load_w = [&](int g) {
        const uint4 *p = reinterpret_cast<const uint4 *>(ws + (int64_t)min(g, last) * wstride);
        return grp{p[0], p[1]};
    };
    auto load_x = [&](int j, int g) {
        if constexpr (XL) {
            // from LDS, the offset through a vector register (the data then
            // counts as per-lane and is waited for where it is used)
            int32_t off = min(g, last) * 32;
            asm("" : "+v"(off));
            const uint4 *p = reinterpret_cast<const uint4 *>(reinterpret_cast<const char *>(xl) + off);
            return grp{p[0], p[1]};
        } else {
            // a per-lane offset keeps the wave-uniform read a vector load
            int64_t off = (int64_t)(j < nc ? j : 0) * a.kp + (int64_t)min(g, last) * 8;
            asm("" : "+v"(off));
            const uint4 *p = reinterpret_cast<const uint4 *>(xs + off);
            return grp{p[0], p[1]};
        }
    };
    acc_ls acc[NC]{};
    uint32_t k_lm = k32_logmask;   // the mask in a register (short encodings)
    asm("" : "+v"(k_lm));
    auto steps = [&](const grp &wq, const grp (&xq)[NC], int u0, int u1) {
        const uint32_t wv[8] = {wq.lo.x, wq.lo.y, wq.lo.z, wq.lo.w, wq.hi.x, wq.hi.y, wq.hi.z, wq.hi.w};
        if constexpr (NC == 1) {
            // one chain per lane: the product of step u + 1 is formed in step
            // u's shadow
            const uint32_t xv[8] = {xq[0].lo.x, xq[0].lo.y, xq[0].lo.z, xq[0].lo.w,
                                    xq[0].hi.x, xq[0].hi.y, xq[0].hi.z, xq[0].hi.w};
            const bool first = u0 < 0;
            const int ub = first ? 0 : u0;
            // the product of step u (x32_mul) as its log and its sign, formed
            // apart: the sign in the first round trip of the step before, the
            // log (the fields added, clamped to the field) in its second
            auto plog = [&](int u) {
                return min(max((wv[u] & k_lm) + (xv[u] & k_lm), k32_one), k32_one + k32_logmask) - k32_one;
            };
            auto psgn = [&](int u) { return (wv[u] ^ xv[u]) & k32_sign; };
            uint32_t tl = ub < u1 ? plog(ub) : 0u, ts = ub < u1 ? psgn(ub) : 0u;
            // uf: the opposite-signs flag (bit 31) of the pending addition
            uint32_t uf = acc[0].s ^ ts;
#pragma unroll
            for (int u = 0; u < 8; u++) {
                if (u >= ub && u < u1) {
                    uint32_t ntl = 0, nts = 0;
                    auto next = [&] {
                        if (u + 1 < u1) nts = psgn(u + 1);
                        return nts;
                    };
                    auto post = [&] {
                        if (u + 1 < u1) ntl = plog(u + 1);
                    };
                    if (first && u == 0) {
                        acc[0] = {tl, ts};
                        uf = ts ^ next();
                        post();
                    } else {
                        uf = x32_add_step(R.O, acc[0], tl, ts, uf, next, post);
                    }
                    tl = ntl;
                    ts = nts;
                }
            }
            return;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (u >= u0 && u < u1) {
#pragma unroll
                for (int j = 0; j < NC; j++) {
                    const uint4 &q = u < 4 ? xq[j].lo : xq[j].hi;
                    const uint32_t xv = (u & 3) == 0 ? q.x : (u & 3) == 1 ? q.y : (u & 3) == 2 ? q.z : q.w;
                    const uint32_t t = x32_mul(wv[u], xv);
                    if (u == 0 && u0 < 0) acc[j] = {t & k32_logmask, t & k32_sign};
                    else x32_add_ls(R.O, acc[j], t & k32_logmask, t & k32_sign);
                }
            }
        }
    };
    {
        grp xq[NC];
#pragma unroll
        for (int j = 0; j < NC; j++) xq[j] = load_x(j, 0);
        const grp wq = load_w(0);
        grp wa[PF], wb[PF], xa[PF][NC], xb[PF][NC];
        auto load_block = [&](grp (&w)[PF], grp (&x)[PF][NC], int g0) {
#pragma unroll
            for (int p = 0; p < PF; p++) {
                w[p] = load_w(g0 + p);
#pragma unroll
                for (int j = 0; j < NC; j++) x[p][j] = load_x(j, g0 + p);
            }
        };
        auto run_block = [&](const grp (&w)[PF], const grp (&x)[PF][NC], int g0) {
#pragma unroll
            for (int p = 0; p < PF; p++)
                if (g0 + p < full) steps(w[p], x[p], 0, 8);
        };
        load_block(wa, xa, 1);
        steps(wq, xq, -1, full > 0 ? 8 : tail);
        for (int g = 1; g < full; g += 2 * PF) {
            load_block(wb, xb, g + PF);
            run_block(wa, xa, g);
            if (g + PF >= full) break;
            load_block(wa, xa, g + 2 * PF);
            run_block(wb, xb, g + PF);
        }
        if (full > 0 && tail > 0) {
            grp tx[NC];
#pragma unroll
            for (int j = 0; j < NC; j++) tx[j] = load_x(j, full);
            steps(load_w(full), tx, 0, tail);
        }
    }
#pragma unroll
    for (int j = 0; j < NC; j++)
        if (j < nc) put(j, x32_to_f32(acc[j].s | acc[j].l));
}

// ---- sequential row sums over LDS --------------------------------------------
// acc <- acc (+) row[i] for i = i0 .. n-1 in order (i0 < n).  row is in LDS,
// 16-byte aligned, and readable up to n rounded up to a whole 16-byte group;
// each group of codes arrives in one 16-byte read issued a group ahead.
// POS: the accumulator and every row[i] are positive (sign bit clear), so the
// xlns32 sum takes the one-round positive addition.
template <class RED, bool POS = false>
__device__ __forceinline__ void chain16(const RED &R, typename RED::acc_t &acc, const uint16_t *row, int i0, int n,
                                        uint32_t &st) {
    const int g0 = i0 >> 3, gl = (n - 1) >> 3;
    auto ld = [&](int g) { return *reinterpret_cast<const uint4 *>(row + 8 * min(g, gl)); };
    auto run = [&](const uint4 &q, int u0, int u1) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (u >= u0 && u < u1) {
                if constexpr (std::is_same<RED, red16<LNSHIP_SUM32>>::value && POS) {
                    acc.l = x32_add_pos(R.O, acc.l, half16(w[u >> 1], u & 1) << 16);
                } else if constexpr (std::is_same<RED, red16<LNSHIP_SUM32>>::value) {
                    const uint32_t v = half16(w[u >> 1], u & 1);
                    R.add_lat(acc, (v & k16_logmask) << 16, (v & k16_sign) << 16, [] {});
                } else if constexpr (POS) {
                    R.add_pos(acc, half16(w[u >> 1], u & 1), st);
                } else {
                    R.add(acc, half16(w[u >> 1], u & 1), st);
                }
            }
    };
    uint4 cur = ld(g0), nxt = ld(g0 + 1);
    run(cur, i0 - 8 * g0, min(n - 8 * g0, 8));
    for (int g = g0 + 1; g < gl; g++) {
        cur = nxt;
        nxt = ld(g + 1);
        run(cur, 0, 8);
    }
    if (gl > g0) run(nxt, 0, n - 8 * gl);
}

// the same over packed xlns32 codes, four per 16-byte group
template <bool POS = false>
__device__ __forceinline__ void chain32(const x32_tab &O, acc_ls &acc, const uint32_t *row, int i0, int n) {
    const int g0 = i0 >> 2, gl = (n - 1) >> 2;
    auto ld = [&](int g) { return *reinterpret_cast<const uint4 *>(row + 4 * min(g, gl)); };
    auto run = [&](const uint4 &q, int u0, int u1) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (u >= u0 && u < u1) {
                if constexpr (POS) acc.l = x32_add_pos(O, acc.l, w[u]);
                else x32_add_desc(O, acc, w[u] & k32_logmask, w[u] & k32_sign, [] {});
            }
    };
    uint4 cur = ld(g0), nxt = ld(g0 + 1);
    run(cur, i0 - 4 * g0, min(n - 4 * g0, 4));
    for (int g = g0 + 1; g < gl; g++) {
        cur = nxt;
        nxt = ld(g + 1);
        run(cur, 0, 4);
    }
    if (gl > g0) run(nxt, 0, n - 4 * gl);
}

// Sums of positive values over the pair image: l <- l (+) row[i] for
// i = i0 .. n-1 in order, as chain32<true> / chain16<..., true> (xlns16 codes
// widened; a sum32 accumulator) compute them.
__device__ __forceinline__ void chain_pos32(const pos_tab &P, uint32_t &l, const uint32_t *row, int i0, int n) {
    const int g0 = i0 >> 2, gl = (n - 1) >> 2;
    auto ld = [&](int g) { return *reinterpret_cast<const uint4 *>(row + 4 * min(g, gl)); };
    auto run = [&](const uint4 &q, int u0, int u1) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int u = 0; u < 4; u++)
            if (u >= u0 && u < u1) l = x32_add_pos2(P, l, w[u]);
    };
    uint4 cur = ld(g0), nxt = ld(g0 + 1);
    run(cur, i0 - 4 * g0, min(n - 4 * g0, 4));
    for (int g = g0 + 1; g < gl; g++) {
        cur = nxt;
        nxt = ld(g + 1);
        run(cur, 0, 4);
    }
    if (gl > g0) run(nxt, 0, n - 4 * gl);
}
__device__ __forceinline__ void chain_pos16(const pos_tab &P, uint32_t &l, const uint16_t *row, int i0, int n) {
    const int g0 = i0 >> 3, gl = (n - 1) >> 3;
    auto ld = [&](int g) { return *reinterpret_cast<const uint4 *>(row + 8 * min(g, gl)); };
    auto run = [&](const uint4 &q, int u0, int u1) {
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int u = 0; u < 8; u++)
            if (u >= u0 && u < u1) l = x32_add_pos2(P, l, half16(w[u >> 1], u & 1) << 16);
    };
    uint4 cur = ld(g0), nxt = ld(g0 + 1);
    run(cur, i0 - 8 * g0, min(n - 8 * g0, 8));
    for (int g = g0 + 1; g < gl; g++) {
        cur = nxt;
        nxt = ld(g + 1);
        run(cur, 0, 8);
    }
    if (gl > g0) run(nxt, 0, n - 8 * gl);
}

// ---- RMS_NORM -------------------------------------------------------------------
// A workgroup takes rb rows: all threads convert and square into LDS, one lane
// per row runs the sequential sum, all threads scale.

template <int MODE>
__global__ __launch_bounds__(k_block) void k_rms16(const float *__restrict__ src, const float *__restrict__ w,
                                                   float *__restrict__ dst, int64_t ncols, int64_t nrows, int rb,
                                                   float eps, uint32_t seed, const uint16_t *state, uint64_t offset,
                                                   dev_tables T) {
    extern __shared__ __align__(16) char lds[];
    pos_tab P{};
    const red16<MODE> R = stage_rows<MODE>(T, lds, P);
    uint16_t *sq = reinterpret_cast<uint16_t *>(lds + ((row_tables_bytes<MODE>() + 15) & ~15));
    __shared__ uint32_t s_inv[64];
    const int64_t r0 = (int64_t)blockIdx.x * rb;
    const int nr = (int)min<int64_t>(rb, nrows - r0);
    const int nc = (int)ncols, nel = nr * nc, rs = (nc + 7) & ~7;   // LDS rows 16-byte aligned
    // element passes in batches of B per thread, loads and lookups issued
    // before the first wait; past the end a thread redoes the last element
    // (the same value to the same place)
    constexpr int B = 8;
    const int nt = (int)blockDim.x;
    for (int e0 = threadIdx.x; e0 < nel; e0 += B * nt) {
        float f[B];
#pragma unroll
        for (int q = 0; q < B; q++) f[q] = src[r0 * ncols + min(e0 + q * nt, nel - 1)];
        uint32_t c[B];
#pragma unroll
        for (int q = 0; q < B; q++) c[q] = x16_from_f32(T.cvt16, f[q]);
#pragma unroll
        for (int q = 0; q < B; q++) {
            const int e = min(e0 + q * nt, nel - 1);
            sq[e + (e / nc) * (rs - nc)] = (uint16_t)x16_mul(c[q], c[q]);
        }
    }
    __syncthreads();
    // every lane of the first wave runs a row's chain, the lanes past the
    // block's rows that of its last row again (only a row's own lane
    // stores): with the wave's other lanes inactive the chain's steps take
    // about 15 % longer
    if (threadIdx.x < 64u) {
        const int r = min((int)threadIdx.x, nr - 1);
        uint32_t s = 0;
        if (MODE == LNSHIP_MONTE)
            s = lfsr_jump(T, monte_start(T, seed, state, offset), (uint64_t)(r0 + r) * (uint64_t)ncols);
        typename red16<MODE>::acc_t acc = R.start(0u, s);
        // squares: positive
        if constexpr (MODE == LNSHIP_SUM32) chain_pos16(P, acc.l, sq + r * rs, 0, nc);
        else chain16<red16<MODE>, true>(R, acc, sq + r * rs, 0, nc, s);
        const uint32_t sum = R.finish(acc) & 0xffffu;
        const uint32_t mean = x16_mul(sum, x16_from_f32(T.cvt16, 1.0f / (float)ncols));
        const uint32_t e16 = x16_from_f32(T.cvt16, eps);
        // the epsilon add is a plain xlns16_add in every mode
        const uint32_t me = x16_add_g(T.gauss16, mean, e16);
        if ((int)threadIdx.x < nr) s_inv[r] = x16_recip(x16_sqrt(me));
    }
    __syncthreads();
    for (int e0 = threadIdx.x; e0 < nel; e0 += B * nt) {
        float f[B];
#pragma unroll
        for (int q = 0; q < B; q++) f[q] = src[r0 * ncols + min(e0 + q * nt, nel - 1)];
        uint32_t c[B];
#pragma unroll
        for (int q = 0; q < B; q++) c[q] = x16_from_f32(T.cvt16, f[q]);
#pragma unroll
        for (int q = 0; q < B; q++) f[q] = T.rev16[x16_mul(c[q], s_inv[min(e0 + q * nt, nel - 1) / nc])];
        if (w) {   // the fused MUL by the weight row, through xlns16 as the MUL node
            float g[B];
#pragma unroll
            for (int q = 0; q < B; q++) g[q] = w[min(e0 + q * nt, nel - 1) % nc];
#pragma unroll
            for (int q = 0; q < B; q++) f[q] = T.rev16[x16_mul(x16_from_f32(T.cvt16, f[q]), x16_from_f32(T.cvt16, g[q]))];
        }
        // only the element's own thread stores (dst may be src)
#pragma unroll
        for (int q = 0; q < B; q++)
            if (e0 + q * nt < nel) dst[r0 * ncols + e0 + q * nt] = f[q];
    }
}

__global__ __launch_bounds__(k_block) void k_rms32(const float *__restrict__ src, const float *__restrict__ w,
                                                   float *__restrict__ dst, int64_t ncols, int64_t nrows, int rb,
                                                   float eps, dev_tables T) {
    extern __shared__ __align__(16) char lds[];
    const pos_tab P = stage_pos32(T, lds);   // every xlns32 addition here adds positive values
    uint32_t *sq = reinterpret_cast<uint32_t *>(lds + k_lds_pos32);
    __shared__ uint32_t s_inv[64];
    const int64_t r0 = (int64_t)blockIdx.x * rb;
    const int nr = (int)min<int64_t>(rb, nrows - r0);
    const int nc = (int)ncols, nel = nr * nc, rs = (nc + 3) & ~3;   // LDS rows 16-byte aligned
    // loads in batches of B per thread (past the end the last element again)
    constexpr int B = 8;
    const int nt = (int)blockDim.x;
    for (int e0 = threadIdx.x; e0 < nel; e0 += B * nt) {
        float f[B];
#pragma unroll
        for (int q = 0; q < B; q++) f[q] = src[r0 * ncols + min(e0 + q * nt, nel - 1)];
#pragma unroll
        for (int q = 0; q < B; q++) {
            const int e = min(e0 + q * nt, nel - 1);
            const uint32_t c = x32_from_f32(f[q]);
            sq[e + (e / nc) * (rs - nc)] = x32_mul(c, c);
        }
    }
    __syncthreads();
    // (all 64 lanes, as in k_rms16)
    if (threadIdx.x < 64u) {
        const int r = min((int)threadIdx.x, nr - 1);
        uint32_t acc = 0u;
        chain_pos32(P, acc, sq + r * rs, 0, nc);   // squares: positive
        const uint32_t mean = x32_mul(acc, x32_from_f32(1.0f / (float)ncols));
        // mean >= 0: the epsilon add is a positive one unless eps < 0
        const uint32_t e = x32_from_f32(eps);
        const uint32_t me = (e & k32_sign) ? x32_add(T.tab32, mean, e) : x32_add_pos2(P, mean, e);
        if ((int)threadIdx.x < nr) s_inv[r] = x32_recip(x32_sqrt(me));
    }
    __syncthreads();
    for (int e0 = threadIdx.x; e0 < nel; e0 += B * nt) {
        float f[B], g[B];
#pragma unroll
        for (int q = 0; q < B; q++) {
            f[q] = src[r0 * ncols + min(e0 + q * nt, nel - 1)];
            g[q] = w ? w[min(e0 + q * nt, nel - 1) % nc] : 0.0f;
        }
        // only the element's own thread stores (dst may be src); with w the
        // fused MUL by the weight row in xlns32, as the MUL node
#pragma unroll
        for (int q = 0; q < B; q++)
            if (e0 + q * nt < nel) {
                float y = x32_to_f32(x32_mul(x32_from_f32(f[q]), s_inv[(e0 + q * nt) / nc]));
                if (w) y = x32_to_f32(x32_mul(x32_from_f32(y), x32_from_f32(g[q])));
                dst[r0 * ncols + e0 + q * nt] = y;
            }
    }
}

// ---- RMS_NORM -> MUL -> MUL_MAT, one activation row, sum32 ----------------------
// The decode graph's h = rms_norm(x) * norm followed by W h, in one launch.
// The mul_mat's chains read h, and h needs the scale, which the rms sum's
// K-step chain gives; so the chains would wait for that chain.  Here they
// start at once, from h formed with a predicted scale, while one lane of a
// fourth wave runs the sum's chain.  The scale is an xlns16 code: the sum32
// sum of the squares, narrowed to xlns16 (1/128 of a binade), then mean,
// epsilon, square root and reciprocal.  The prediction sums the squares'
// values in F32 and rounds the log to the nearest xlns16 step: that is the
// narrowed sum unless the sum lies within the xlns32 chain's error (and the
// F32 sum's) of a rounding boundary.  When the chain's scale differs from the predicted one,
// h is formed again from it and the chains run again, so the output is that
// of the three nodes in every case.
constexpr int k_rms_mm_rows = 3 * 64;   // chain lanes per workgroup (waves 0-2; wave 3 sums)

// W: rows per chain wave (64, or 16 with the other lanes idle during the
// chains, as in k_mm16)
template <int PF, int W = 64>
__global__ __launch_bounds__(k_block) void k_mm16_rms(mm_args16 a, dev_tables T) {
    static_assert(k_block == k_rms_mm_rows + 64, "three chain waves and the sum's wave");
    extern __shared__ __align__(16) char lds[];
    if (blockIdx.x & ((1u << a.xcd_sh) - 1u)) return;   // as in k_mm16
    const int lane = (int)(threadIdx.x & 63u);
    const int64_t m = (int64_t)(blockIdx.x >> a.xcd_sh) * (3 * W) + (threadIdx.x >> 6) * W + lane;
    const bool active = threadIdx.x < k_rms_mm_rows && lane < W && m < a.M;
    // the chain's first weights before the tables (as in k_mm16)
    mm_head<PF> hw{};
    if (active) hw = mm16_head<PF>(a, m, 0);
    const red16<LNSHIP_SUM32> R = stage_for<LNSHIP_SUM32, true>(T, lds);
    const int K = (int)a.K, kp = (int)a.kp;
    uint16_t *xl = reinterpret_cast<uint16_t *>(lds + mm_xl_offset<LNSHIP_SUM32>());   // h, as the chains read it
    uint16_t *sq = xl + kp + k_xl_pad / 2;                                              // the squares of x
    __shared__ float s_part[k_block / 64];
    __shared__ uint32_t s_inv[2];   // the predicted scale, the chain's
    // the squares of x's codes into LDS (the sum's addends), their values
    // summed per wave (in F32: the prediction only has to land on the
    // chain's xlns16 step, 1/128 of a binade, and a miss costs a rerun).
    // The codes of x and of the norm row for k < RK k_block stay in
    // registers for forming h (past that they are formed again there).
    constexpr int RK = 4;
    uint32_t cxr[RK], cnr[RK];
    float part = 0.0f;
    auto square = [&](int k, uint32_t c) {
        const uint32_t q = x16_mul(c, c);
        part += exp2f((float)((int)(q & k16_logmask) - (int)k16_one) * (1.0f / 128.0f));
        sq[k] = (uint16_t)q;
    };
#pragma unroll
    for (int i = 0; i < RK; i++) {
        const int k = (int)threadIdx.x + i * k_block;
        cxr[i] = k < K ? x16_from_f32(T.cvt16, a.xf[k]) : 0u;
        cnr[i] = k < K ? x16_from_f32(T.cvt16, a.norm[k]) : 0u;
    }
#pragma unroll
    for (int i = 0; i < RK; i++) {
        const int k = (int)threadIdx.x + i * k_block;
        if (k < K) square(k, cxr[i]);
        else if (k < kp) sq[k] = 0;
    }
    for (int k = (int)threadIdx.x + RK * k_block; k < kp; k += k_block) {
        if (k < K) square(k, x16_from_f32(T.cvt16, a.xf[k]));
        else sq[k] = 0;
    }
    for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o);
    if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = part;
    __syncthreads();
    // the scale from the narrowed sum (the rms_norm node's tail, as k_rms16;
    // the codes of 1 / K and eps come from the host's conversion table)
    auto scale_of = [&](uint32_t sum) {
        const uint32_t mean = x16_mul(sum, a.rms_ik);
        return x16_recip(x16_sqrt(x16_add_g(T.gauss16, mean, a.rms_eps)));
    };
    if (threadIdx.x == 0) {
        float S = 0.0f;
        for (int i = 0; i < k_block / 64; i++) S += s_part[i];
        // the nearest xlns16 code of S, within the code range
        const float l = S > 0.0f ? floorf(log2f(S) * 128.0f + 0.5f) + (float)k16_one : 0.0f;
        const uint32_t sum = (uint32_t)fminf(fmaxf(l, 0.0f), (float)k16_logmask);
        s_inv[0] = (scale_of(sum) + a.skew) & 0xffffu;
    }
    __syncthreads();
    // h = the MUL node's output from the rms_norm node's, each through F32
    // as between graph nodes (rho16: cvt16 of rev16), then into xlns16 as
    // the mul_mat converts its activations (k past K: zero)
    auto stage_h = [&](uint32_t inv) {
#pragma unroll
        for (int i = 0; i < RK; i++) {
            const int k = (int)threadIdx.x + i * k_block;
            if (k < kp) xl[k] = k < K ? (uint16_t)T.rho16[x16_mul(T.rho16[x16_mul(cxr[i], inv)], cnr[i])] : 0;
        }
        for (int k = (int)threadIdx.x + RK * k_block; k < kp; k += k_block) {
            uint32_t h = 0;
            if (k < K) {
                const uint32_t y = T.rho16[x16_mul(x16_from_f32(T.cvt16, a.xf[k]), inv)];
                h = T.rho16[x16_mul(y, x16_from_f32(T.cvt16, a.norm[k]))];
            }
            xl[k] = (uint16_t)h;
        }
    };
    uint32_t inv = s_inv[0];
    stage_h(inv);
    __syncthreads();
    uint32_t res[1] = {0};
    // pass 0 with the predicted scale; a second pass only when the chain's
    // scale differs (every thread reads the same two words after the barrier)
    for (int pass = 0;; pass++) {
        if (active) {
            mm16_chains<LNSHIP_SUM32, 1, PF, true, true>(a, T, R, xl, m, 0, 0, 0, 0, 1, res, hw);
        } else if (pass == 0 && threadIdx.x == k_rms_mm_rows) {
            uint32_t st = 0;
            typename red16<LNSHIP_SUM32>::acc_t acc = R.start(0u, st);
            chain16<red16<LNSHIP_SUM32>, true>(R, acc, sq, 0, K, st);   // squares: positive
            s_inv[1] = scale_of(R.finish(acc) & 0xffffu);
        }
        __syncthreads();
        const uint32_t want = s_inv[1];
        if (want == inv) break;
        inv = want;
        stage_h(inv);
        __syncthreads();
    }
    if (active) a.dst[m] = T.rev16[res[0]];
}

// ---- SOFT_MAX -------------------------------------------------------------------
// A workgroup takes rb rows: scale / mask / row maximum (order-free: canonical
// order is total) and exp in parallel, one lane per row sums in element order,
// then the division in parallel.

struct sm_args {
    const float *src;
    const float *mask;
    float *dst;
    int64_t n, ne1, ne2, ne3;
    int64_t mne0, mne1, mne2, mne3;
    float scale;
    uint32_t seed;
    int rb;
    const uint16_t *state;   // Monte start read on the device (null: seed)
    uint64_t offset;
};

__device__ __forceinline__ const float *mask_row(const sm_args &a, int64_t row) {
    const int64_t i1 = row % a.ne1, i2 = (row / a.ne1) % a.ne2, i3 = row / (a.ne1 * a.ne2);
    return a.mask + (((i3 % a.mne3) * a.mne2 + (i2 % a.mne2)) * a.mne1 + i1) * a.mne0;
}

template <int MODE>
__global__ __launch_bounds__(k_block) void k_softmax16(sm_args a, dev_tables T) {
    extern __shared__ __align__(16) char lds[];
    pos_tab P{};
    const red16<MODE> R = stage_rows<MODE>(T, lds, P);
    // the plain xlns16 adder (scale, mask bias, max subtraction) reads the
    // global copy of the Gaussian-log table
    uint16_t *c = reinterpret_cast<uint16_t *>(lds + ((row_tables_bytes<MODE>() + 15) & ~15));
    __shared__ int32_t s_max[64];
    __shared__ uint32_t s_tot[64];
    __shared__ const float *s_mrow[64];
    __shared__ int s_last[64];   // a row's last element with a nonzero exp
    const int64_t r0 = (int64_t)blockIdx.x * a.rb;
    const int nr = (int)min<int64_t>(a.rb, a.ne1 * a.ne2 * a.ne3 - r0);
    const int n = (int)a.n, nel = nr * n;   // a row fits in LDS, so 32-bit counts suffice
    const int rs = (n + 7) & ~7;            // LDS rows 16-byte aligned
    if ((int)threadIdx.x < nr) {
        s_last[threadIdx.x] = 0;
        s_max[threadIdx.x] = x16_canon(0xffffu);
        s_mrow[threadIdx.x] = a.mask ? mask_row(a, r0 + threadIdx.x) : nullptr;
    }
    __syncthreads();
    const uint32_t sc = x16_from_f32(T.cvt16, a.scale);
    const bool has_mask = a.mask != nullptr;
    // The element passes run in batches of B elements per thread, branch
    // free: every load and table lookup of a batch is issued before the first
    // one is waited for.  Past the end a thread redoes the last element (the
    // same value to the same place).
    constexpr int B = 8;
    const int nt = (int)blockDim.x;
    for (int e0 = threadIdx.x; e0 < nel; e0 += B * nt) {
        int r[B], o[B];
        float f[B], mf[B];
#pragma unroll
        for (int q = 0; q < B; q++) {
            const int e = min(e0 + q * nt, nel - 1);
            r[q] = e / n;
            const int i = e - r[q] * n;
            o[q] = e + r[q] * (rs - n);
            f[q] = a.src[(r0 + r[q]) * a.n + i];
            mf[q] = has_mask ? s_mrow[r[q]][i] : 0.0f;
        }
        uint32_t v[B], mk[B];
#pragma unroll
        for (int q = 0; q < B; q++) {
            v[q] = x16_from_f32(T.cvt16, f[q]);
            mk[q] = x16_from_f32(T.cvt16, mf[q]);
        }
        uint32_t vm[B], va[B];
#pragma unroll
        for (int q = 0; q < B; q++) {
            vm[q] = x16_mul(v[q], sc);
            va[q] = x16_add_g(T.gauss16, vm[q], mk[q]);
        }
#pragma unroll
        for (int q = 0; q < B; q++) asm volatile("" ::"v"(va[q]));
#pragma unroll
        for (int q = 0; q < B; q++) {
            const bool masked_out = has_mask && (mf[q] <= -3.0e38f || mk[q] == 0xffffu);
            const uint32_t w = v[q] == 0xffffu || masked_out ? 0xffffu : (has_mask && (mk[q] & k16_logmask)) ? va[q] : vm[q];
            c[o[q]] = (uint16_t)w;
            atomicMax(&s_max[r[q]], x16_canon(w));
        }
    }
    __syncthreads();
    for (int e0 = threadIdx.x; e0 < nel; e0 += B * nt) {
        int o[B];
        uint32_t mx[B], cv[B], sh[B];
#pragma unroll
        for (int q = 0; q < B; q++) {
            const int e = min(e0 + q * nt, nel - 1), r = e / n;
            const int32_t cm = s_max[r];
            mx[q] = (uint32_t)(uint16_t)(cm < 0 ? (cm ^ 0x7fff) : cm);
            o[q] = e + r * (rs - n);
            cv[q] = c[o[q]];
        }
#pragma unroll
        for (int q = 0; q < B; q++) sh[q] = x16_add_g(T.gauss16, cv[q], mx[q] ^ k16_sign);
#pragma unroll
        for (int q = 0; q < B; q++) sh[q] = T.exp16[sh[q]];
        // in place: only the element's own thread writes it (a thread that
        // redoes the last element may read it after its owner wrote it)
#pragma unroll
        for (int q = 0; q < B; q++)
            if (e0 + q * nt < nel) {
                c[o[q]] = (uint16_t)sh[q];
                if (sh[q] & k16_logmask) {
                    const int e = e0 + q * nt, r = e / n;
                    atomicMax(&s_last[r], e - r * n);
                }
            }
    }
    __syncthreads();
    // (all 64 lanes, as in k_rms16)
    if (threadIdx.x < 64u) {
        const int r = min((int)threadIdx.x, nr - 1);
        uint32_t s = 0;
        if (MODE == LNSHIP_MONTE)
            s = lfsr_jump(T, monte_start(T, a.seed, a.state, a.offset), (uint64_t)(r0 + r) * (uint64_t)(a.n - 1));
        const uint16_t *row = c + r * rs;
        typename red16<MODE>::acc_t acc = R.start(row[0], s);
        // The entries after the row's last nonzero exp lie after its maximum
        // (whose exp, 1, is nonzero), so the running sum there is at least 1;
        // each of them is an exp of log 0 (masked or underflowed), which every
        // mode's adder (as restated here) adds as nothing at a distance of 2^14
        // and more.  So the chain stops at the last nonzero exp (Monte: the
        // draws after it are not taken; the next op's start does not depend
        // on them)
        const int n_eff = s_last[r] + 1;
        if (n_eff > 1) {   // exps: positive
            if constexpr (MODE == LNSHIP_SUM32) chain_pos16(P, acc.l, row, 1, n_eff);
            else chain16<red16<MODE>, true>(R, acc, row, 1, n_eff, s);
        }
        if ((int)threadIdx.x < nr) s_tot[r] = R.finish(acc) & 0xffffu;
    }
    __syncthreads();
    for (int e0 = threadIdx.x; e0 < nel; e0 += B * nt) {
        uint32_t y[B];
#pragma unroll
        for (int q = 0; q < B; q++) {
            const int e = min(e0 + q * nt, nel - 1), r = e / n;
            y[q] = x16_div(c[e + r * (rs - n)], s_tot[r]);
        }
        float out[B];
#pragma unroll
        for (int q = 0; q < B; q++) out[q] = T.rev16[y[q]];
#pragma unroll
        for (int q = 0; q < B; q++) a.dst[r0 * a.n + min(e0 + q * nt, nel - 1)] = out[q];
    }
}

// ---- elementwise ops of the Llama graph ---------------------------------------

// The elementwise ops in either format: fmt16 (xlns16 through the
// conversion, decode, Gaussian-log and sigmoid tables) or fmt32 (xlns32,
// converted arithmetically, adder over the global xlns32 tables).
struct fmt16 {
    using code_t = uint16_t;
    const dev_tables &T;
    __device__ __forceinline__ uint32_t from(float v) const { return x16_from_f32(T.cvt16, v); }
    __device__ __forceinline__ float to(uint32_t c) const { return T.rev16[c]; }
    __device__ __forceinline__ uint32_t add(uint32_t x, uint32_t y) const { return x16_add_g(T.gauss16, x, y); }
    __device__ __forceinline__ uint32_t mul(uint32_t x, uint32_t y) const { return x16_mul(x, y); }
    __device__ __forceinline__ uint32_t neg(uint32_t x) const { return x ^ k16_sign; }
    // xlns16_silu: x times the table sigmoid of x
    __device__ __forceinline__ uint32_t silu(uint32_t x) const { return x16_mul(x, T.sig16[x]); }
};
struct fmt32 {
    using code_t = uint32_t;
    const dev_tables &T;
    __device__ __forceinline__ uint32_t from(float v) const { return x32_from_f32(v); }
    __device__ __forceinline__ float to(uint32_t c) const { return x32_to_f32(c); }
    __device__ __forceinline__ uint32_t add(uint32_t x, uint32_t y) const { return x32_add(T.tab32, x, y); }
    __device__ __forceinline__ uint32_t mul(uint32_t x, uint32_t y) const { return x32_mul(x, y); }
    __device__ __forceinline__ uint32_t neg(uint32_t x) const { return x ^ k32_sign; }
    __device__ __forceinline__ uint32_t silu(uint32_t x) const { return x32_silu(x); }
};
template <int W>
using fmt_t = typename std::conditional<W == 16, fmt16, fmt32>::type;

template <int W, int OP>   // OP 0 add, 1 mul
__global__ void k_binary(const float *__restrict__ a, const float *__restrict__ b, int64_t n, int64_t nb,
                         float *__restrict__ dst, dev_tables T) {
    const fmt_t<W> F{T};
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        const uint32_t x = F.from(a[i]), y = F.from(b[i % nb]);
        dst[i] = F.to(OP == 0 ? F.add(x, y) : F.mul(x, y));
    }
}

template <int W>
__global__ void k_swiglu(const float *__restrict__ g, int64_t g_ld, const float *__restrict__ u, int64_t u_ld,
                         float *__restrict__ dst, int64_t ncols, int64_t nrows, dev_tables T) {
    const fmt_t<W> F{T};
    const int64_t n = ncols * nrows;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        const int64_t r = i / ncols, c = i - r * ncols;
        const uint32_t gv = F.from(g[r * g_ld + c]);
        const uint32_t uv = F.from(u[r * u_ld + c]);
        dst[i] = F.to(F.mul(F.silu(gv), uv));
    }
}

// y = x s (+ b when b is not zero), in the format's arithmetic
template <int W>
__global__ void k_scale(const float *__restrict__ src, float *__restrict__ dst, int64_t n, float s, float b,
                        dev_tables T) {
    const fmt_t<W> F{T};
    const uint32_t sc = F.from(s), bc = F.from(b);
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        uint32_t v = F.mul(F.from(src[i]), sc);
        if (b != 0.0f) v = F.add(v, bc);
        dst[i] = F.to(v);
    }
}

__global__ void k_get_rows_packed(const uint16_t *__restrict__ w, int64_t K, int64_t M, const int32_t *__restrict__ rows,
                                  int64_t nrows, float *__restrict__ dst, const float *__restrict__ rev) {
    const int64_t n = nrows * K;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        const int64_t r = i / K, k = i - r * K;
        const int64_t m = rows[r];
        dst[i] = rev[w[((k >> 3) * M + m) * 8 + (k & 7)]];
    }
}

// one thread per rotated pair (or passthrough element)
template <class F>
__device__ __forceinline__ void rope_pair(const F &f, const float *xr, int64_t j, int n_dims, int neox, const float *cs,
                                          int64_t &i0, int64_t &i1, uint32_t &r0, uint32_t &r1) {
    const uint32_t c = f.from(cs[j * 2]), sn = f.from(cs[j * 2 + 1]);
    i0 = neox ? j : 2 * j;
    i1 = neox ? j + n_dims / 2 : 2 * j + 1;
    const uint32_t x0 = f.from(xr[i0]), x1 = f.from(xr[i1]);
    r0 = f.add(f.mul(x0, c), f.neg(f.mul(x1, sn)));
    r1 = f.add(f.mul(x0, sn), f.mul(x1, c));
}

// item i of a rope: a rotated pair (j < n_dims / 2) or a passthrough element
// of row (token, head); ntok * nhead * (n_dims / 2 + ne0 - n_dims) items
template <class F>
__device__ __forceinline__ void rope_item(const F &f, int64_t i, const float *x, int64_t x_ld, const int32_t *pos,
                                          int64_t nhead, int64_t ne0, int n_dims, int neox, const float *cos_sin,
                                          float *dst) {
    const int64_t half = n_dims / 2, per = half + (ne0 - n_dims);
    const int64_t row = i / per, j = i - row * per;
    const int64_t t = row / nhead, h = row - t * nhead;
    const float *xr = x + t * x_ld + h * ne0;
    float *yr = dst + (t * nhead + h) * ne0;
    if (j < half) {
        int64_t i0, i1;
        uint32_t r0, r1;
        rope_pair(f, xr, j, n_dims, neox, cos_sin + (int64_t)pos[t] * half * 2, i0, i1, r0, r1);
        yr[i0] = f.to(r0);
        yr[i1] = f.to(r1);
    } else {
        const int64_t i0 = n_dims + (j - half);
        yr[i0] = f.to(f.from(xr[i0]));
    }
}

template <int W>
__global__ void k_rope(const float *__restrict__ x, int64_t x_ld, const int32_t *__restrict__ pos, int64_t ntok,
                       int64_t nhead, int64_t ne0, int n_dims, int neox, const float *__restrict__ cos_sin,
                       float *__restrict__ dst, dev_tables T) {
    const fmt_t<W> F{T};
    const int64_t n = ntok * nhead * (n_dims / 2 + (ne0 - n_dims));
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x)
        rope_item(F, i, x, x_ld, pos, nhead, ne0, n_dims, neox, cos_sin, dst);
}

// F32 value -> IEEE half (round to nearest even) -> F32 -> LNS, as the KV
// cache stores and reads it
// item i (element (token, head, d)) of a KV-cache store;
// ntok * nhead * ne0 items
// A position outside the cache's cache_m rows is recorded (err, as an index
// out of range) and its item is skipped: nothing is read from the rope
// table or written to the cache for it.
template <class F, class C>
__device__ __forceinline__ void store_kv_item(const F &f, int64_t i, const float *x, int64_t x_ld, const int32_t *pos,
                                              int64_t nhead, int64_t ne0, int rope_n_dims, const float *cos_sin,
                                              C *cache, int64_t cache_m, int64_t cache_slice, int transposed,
                                              const int32_t *seq, int64_t seq_stride, unsigned long long *err) {
    const int64_t half = rope_n_dims / 2;
    const int64_t row = i / ne0, d = i - row * ne0;
    const int64_t t = row / nhead, h = row - t * nhead;
    const float *xr = x + t * x_ld + h * ne0;
    const int64_t p = pos[t];
    if (p < 0 || p >= cache_m) {
        index_fault(err, p);
        return;
    }
    float v;
    if (rope_n_dims > 0 && d < rope_n_dims) {
        // normal rope: element d belongs to pair d / 2
        int64_t i0, i1;
        uint32_t r0, r1;
        rope_pair(f, xr, d / 2, rope_n_dims, 0, cos_sin + p * half * 2, i0, i1, r0, r1);
        v = f.to((d & 1) ? r1 : r0);
    } else if (rope_n_dims > 0) {
        v = f.to(f.from(xr[d]));
    } else {
        v = xr[d];
    }
    const int64_t o = transposed ? h * cache_slice + ((p >> 3) * ne0 + d) * 8 + (p & 7)
                                 : h * cache_slice + ((d >> 3) * cache_m + p) * 8 + (d & 7);
    cache[(seq ? (int64_t)seq[t] * seq_stride : 0) + o] = (C)f.from(__half2float(__float2half_rn(v)));
}

template <int W>
__global__ void k_store_kv(const float *__restrict__ x, int64_t x_ld, const int32_t *__restrict__ pos, int64_t ntok,
                           int64_t nhead, int64_t ne0, int rope_n_dims, const float *__restrict__ cos_sin,
                           typename fmt_t<W>::code_t *__restrict__ cache, int64_t cache_m, int64_t cache_slice,
                           int transposed, const int32_t *__restrict__ seq, int64_t seq_stride, dev_tables T,
                           unsigned long long *err) {
    const fmt_t<W> F{T};
    const int64_t n = ntok * nhead * ne0;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x)
        store_kv_item(F, i, x, x_ld, pos, nhead, ne0, rope_n_dims, cos_sin, cache, cache_m, cache_slice, transposed,
                      seq, seq_stride, err);
}

// The query rope and the key / value cache stores after a fused QKV
// mul_mat, as one grid: items [0, nq) rope the query heads, the next nk
// store the (rotated) key heads, the last nk the value heads.
template <int W>
__global__ void k_rope_store_kv(lnship_qkv_store_args a, dev_tables T, unsigned long long *err) {
    using C = typename fmt_t<W>::code_t;
    const fmt_t<W> F{T};
    const int64_t hd = a.head_dim, nd = a.rope_n_dims;
    const int64_t nq = a.ntok * a.n_head * (nd / 2 + (hd - nd)), nk = a.ntok * a.n_head_kv * hd;
    const float *xk = a.qkv + a.n_head * hd, *xv = xk + a.n_head_kv * hd;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nq + 2 * nk;
         i += (int64_t)blockDim.x * gridDim.x) {
        if (i < nq) {
            // the rope table has cache_m rows: a query beyond them is recorded
            // and skipped, like the cache stores
            const int64_t t = i / (a.n_head * (nd / 2 + (hd - nd)));
            const int64_t p = a.pos[t];
            if (p < 0 || p >= a.cache_m) index_fault(err, p);
            else rope_item(F, i, a.qkv, a.qkv_ld, a.pos, a.n_head, hd, (int)nd, 0, a.cos_sin, a.q_dst);
        } else if (i < nq + nk) {
            store_kv_item(F, i - nq, xk, a.qkv_ld, a.pos, a.n_head_kv, hd, (int)nd, a.cos_sin, (C *)a.k_cache,
                          a.cache_m, a.k_slice, 0, a.seq, a.seq_stride, err);
        } else {
            store_kv_item(F, i - nq - nk, xv, a.qkv_ld, a.pos, a.n_head_kv, hd, 0, a.cos_sin, (C *)a.v_cache,
                          a.cache_m, a.v_slice, 1, a.seq, a.seq_stride, err);
        }
    }
}

// ggml views on the device: element (i0, i1, i2, i3) at byte offset
// i0 nb0 + i1 nb1 + i2 nb2 + i3 nb3, gathered into (or scattered from) a
// contiguous F32 array in ggml element order.
struct strided4 {
    int64_t ne[4];
    int64_t nb[4];
};

template <int SRC_HALF>
__global__ void k_gather_f32(const char *__restrict__ src, strided4 g, float *__restrict__ dst) {
    const int64_t n = g.ne[0] * g.ne[1] * g.ne[2] * g.ne[3];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        int64_t r = i;
        const int64_t i0 = r % g.ne[0];
        r /= g.ne[0];
        const int64_t i1 = r % g.ne[1];
        r /= g.ne[1];
        const int64_t i2 = r % g.ne[2], i3 = r / g.ne[2];
        const char *p = src + i0 * g.nb[0] + i1 * g.nb[1] + i2 * g.nb[2] + i3 * g.nb[3];
        dst[i] = SRC_HALF ? __half2float(*reinterpret_cast<const __half *>(p)) : *reinterpret_cast<const float *>(p);
    }
}

__global__ void k_scatter_f32(const float *__restrict__ src, char *__restrict__ dst, strided4 g) {
    const int64_t n = g.ne[0] * g.ne[1] * g.ne[2] * g.ne[3];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        int64_t r = i;
        const int64_t i0 = r % g.ne[0];
        r /= g.ne[0];
        const int64_t i1 = r % g.ne[1];
        r /= g.ne[1];
        const int64_t i2 = r % g.ne[2], i3 = r / g.ne[2];
        *reinterpret_cast<float *>(dst + i0 * g.nb[0] + i1 * g.nb[1] + i2 * g.nb[2] + i3 * g.nb[3]) = src[i];
    }
}

// ---- decode attention: KQ, soft_max and KQV of one token in one launch ------
// head_dim up to which the KQV chain may stop at the last nonzero exp
constexpr int k_attn_tail_hd = 256;
// The decode attention's workgroups avoid XCD 0, where the co-located decode
// GEMVs before them run (workgroups are dealt to the eight XCDs round-robin,
// block b to XCD b mod 8): measured with cycle stamps, a head's chains on the
// XCD of the preceding GEMVs ran about 13 % longer than on any other (moving
// the GEMVs to XCD 1 moved the slow head there), and the launch waits for its
// slowest head.  Block b (b mod 8 != 0) works as head b - b / 8 - 1; the
// grid (attn_grid) ends at the block of the last head.
__device__ __forceinline__ int attn_head(bool &idle) {
    idle = (blockIdx.x & 7u) == 0;
    return (int)(blockIdx.x - blockIdx.x / 8u - 1u);
}

struct attn_args {
    const float *q;
    const uint16_t *k, *v;
    int64_t k_gs, k_slice, v_gs, v_slice;   // codes between groups of eight; between kv heads
    const float *mask;
    float scale;
    float *dst;
    int hd, n_kv, rep;   // head_dim, cells, query heads per kv head
    uint32_t skew;       // added to the predicted soft_max total (0; a test hook sets it)
    // The query rope and the current cell's cache stores folded in
    // (lnship16_rope_attn_decode); qkv null: q holds the rotated queries and
    // the caches hold the cell (lnship16_attn_decode)
    const float *qkv;              // [n_head + 2 n_head_kv][hd] F32: the fused QKV product of the token
    const int32_t *pos;            // [1] the token's position, device
    const float *cos_sin;          // the rope table (lnship_rope_table layout)
    int rope_n_dims, nh, nhkv;     // rotated dims; query and kv heads
    unsigned long long *err;       // a position outside the cache is recorded here
    // lnship16_attn_decode_seqs: nseq sequences, workgroup head hh = s nh + h
    // (nh is set for every launch); Monte: the kq, soft_max and kqv nodes'
    // starts, monte_start of (mseed[i], mstate, moff[i])
    int nseq;
    uint32_t mseed[3];
    const uint16_t *mstate;
    uint64_t moff[3];
    // with qkv: floats between the QKV rows of consecutive sequences (row s
    // is sequence s's token, at position pos[s], its cells in the caches at
    // s nhkv k_slice and s nhkv v_slice, where the attention reads them)
    int64_t qld;
};

// The rope of head h's query of sequence sqn into xq (its xlns16 codes,
// through F32 as the ROPE node writes them and the kq mul_mat converts them)
// and the stores of kv head kv's rotated key and value of that sequence's
// current cell, exactly as k_rope_store_kv makes them for its token.  Every
// query head of a kv group stores that group's cell, with the same codes,
// before its chains read the caches.  false (nothing done, the fault
// recorded) for a position outside the cache.
__device__ __forceinline__ bool attn_rope_store(const attn_args &a, const dev_tables &T, int h, int kv, int sqn,
                                                uint16_t *xq) {
    const fmt16 F{T};
    const int hd = a.hd, nd = a.rope_n_dims, half = nd / 2;
    const int64_t cache_m = a.k_gs / 8;
    const int32_t *pos = a.pos + sqn;
    const int64_t p = pos[0];
    if (p < 0 || p >= cache_m) {
        if (threadIdx.x == 0) index_fault(a.err, p);
        return false;
    }
    const float *row = a.qkv + (int64_t)sqn * a.qld;
    const float *xk = row + (int64_t)a.nh * hd, *xv = xk + (int64_t)a.nhkv * hd;
    uint16_t *kc = const_cast<uint16_t *>(a.k) + (int64_t)sqn * a.nhkv * a.k_slice;
    uint16_t *vc = const_cast<uint16_t *>(a.v) + (int64_t)sqn * a.nhkv * a.v_slice;
    for (int i = threadIdx.x; i < 2 * hd; i += blockDim.x) {
        if (i < hd)
            store_kv_item(F, (int64_t)kv * hd + i, xk, a.qld, pos, a.nhkv, hd, nd, a.cos_sin, kc, cache_m, a.k_slice,
                          0, (const int32_t *)nullptr, 0, a.err);
        else
            store_kv_item(F, (int64_t)kv * hd + (i - hd), xv, a.qld, pos, a.nhkv, hd, 0, a.cos_sin, vc, cache_m,
                          a.v_slice, 1, (const int32_t *)nullptr, 0, a.err);
    }
    const float *xr = row + (int64_t)h * hd, *cs = a.cos_sin + p * half * 2;
    for (int j = threadIdx.x; j < half + (hd - nd); j += blockDim.x) {
        if (j < half) {
            int64_t i0, i1;
            uint32_t r0, r1;
            rope_pair(F, xr, j, nd, 0, cs, i0, i1, r0, r1);
            xq[i0] = (uint16_t)F.from(F.to(r0));
            xq[i1] = (uint16_t)F.from(F.to(r1));
        } else {
            const int i0 = nd + (j - half);
            xq[i0] = (uint16_t)F.from(F.to(F.from(xr[i0])));
        }
    }
    for (int k = hd + threadIdx.x; k < ((hd + 7) & ~7); k += blockDim.x) xq[k] = 0;
    return true;
}

// Terms k0 <= k < k1 of one output of a GEMV over weights in the packed
// layout (the row's groups of eight codes gs codes apart from w, the
// activations' codes at x in LDS), each an xlns16_mul product, added into acc
// in k order as k_mm16 adds them (term 0 starts acc).  The weights of the next
// PF groups are in flight while a block is added.
// row_chain for sum32, in the order and with the pipeline of k_mm16's
// single-chain loop: the products of steps 2i and 2i + 1 are formed together
// (the two 16-bit halves of one word) in the second round trip of an earlier
// step, each step's product is unpacked from its pair in the first round
// trip of the step before it, which also passes on the opposite-signs flag.
// Groups strictly inside [k0, k1) run their eight steps with no bounds test;
// only the first and the last group test each step.
__device__ __forceinline__ void row_chain_x32(const red16<LNSHIP_SUM32> &R, acc_ls &acc,
                                              const uint16_t *__restrict__ w, int64_t gs, const uint16_t *x, int k0,
                                              int k1) {
    if (k1 <= k0) return;
    constexpr int PF = 4;
    const int gf = k0 >> 3, gl = (k1 - 1) >> 3;
    const int uf = k0 & 7, ul = k1 - 8 * gl;   // the first group's first step, the last group's end
    // masks in registers (short encodings of the instructions that take them)
    uint32_t k_lm = 0x7fff7fffu, k_sg = k32_sign, k_hi = 0xffff0000u;
    asm("" : "+v"(k_lm), "+v"(k_sg), "+v"(k_hi));
    // two xlns16 products (xlns16_mul) in the halves of one word: the log
    // fields added (no carry crosses the halves), less the offset with
    // unsigned saturation (underflow: log 0), capped at 0x7fff; signs xor'ed
    auto pair = [&](uint32_t wv, uint32_t xv, uint32_t &l, uint32_t &sg) {
        const uint32_t lm = (wv & k_lm) + (xv & k_lm);
        l = pk_min_u16(pk_sub_sat_u16(lm, 0x40004000u), 0x7fff7fffu);
        sg = wv ^ xv;
    };
    // the product of step u at the xlns32 positions, from its pair
    auto half = [&](int u, uint32_t l, uint32_t sg, uint32_t &tl, uint32_t &ts) {
        if ((u & 1) == 0) {
            tl = l << 16;
            ts = (sg << 16) & k_sg;
        } else {
            tl = l & k_hi;
            ts = sg & k_sg;
        }
    };
    // carried between groups: the pending step's product and flag, and the
    // next group's first pair
    uint32_t c_tl = 0, c_ts = 0, c_uf = 0, c_pl = 0, c_ps = 0;
    // steps [u0, u1) of a group (wq, xq); wn, xn: the next group's data.
    // fresh: the group's pairs are formed here (the chain's first group);
    // start: its step u0 = 0 is term 0, which starts the sum
    auto group = [&](const uint4 &wq, const uint4 &xq, const uint4 &wn, const uint4 &xn, int u0, int u1, bool fresh,
                     bool start) __attribute__((always_inline)) {
        const uint32_t ww[4] = {wq.x, wq.y, wq.z, wq.w}, xx[4] = {xq.x, xq.y, xq.z, xq.w};
        uint32_t pl[4], ps[4];
        if (fresh) {
#pragma unroll
            for (int i = 0; i < 4; i++) pair(ww[i], xx[i], pl[i], ps[i]);
            pair(wn.x, xn.x, c_pl, c_ps);
#pragma unroll
            for (int u = 0; u < 8; u++)
                if (u == u0) half(u, pl[u >> 1], ps[u >> 1], c_tl, c_ts);
            c_uf = acc.s ^ c_ts;
        } else {
            pl[0] = c_pl;
            ps[0] = c_ps;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (u >= u0 && u < u1) {
                uint32_t ntl = 0, nts = 0;
                auto next = [&] {
                    if (u + 1 < u1) half(u + 1, pl[(u + 1) >> 1], ps[(u + 1) >> 1], ntl, nts);
                    else if (u == 7) half(0, c_pl, c_ps, ntl, nts);
                    return nts;
                };
                // a fresh group has every pair already
                auto post = [&] {
                    if (fresh) return;
                    if ((u & 1) == 0 && u < 6) pair(ww[(u >> 1) + 1], xx[(u >> 1) + 1], pl[(u >> 1) + 1], ps[(u >> 1) + 1]);
                    if (u == 6) pair(wn.x, xn.x, c_pl, c_ps);
                };
                if (start && u == 0) {
                    acc = {c_tl, c_ts};
                    c_uf = c_ts ^ next();
                    post();
                } else {
                    c_uf = x32_add_step(R.O, acc, c_tl, c_ts, c_uf, next, post);
                }
                c_tl = ntl;
                c_ts = nts;
            }
        }
    };
    // a group of the block loop: the last one tests its steps, the others
    // run all eight
    auto body = [&](const uint4 &wq, const uint4 &xq, const uint4 &wn, const uint4 &xn, int g)
                    __attribute__((always_inline)) {
        if (g < gl) group(wq, xq, wn, xn, 0, 8, false, false);
        else group(wq, xq, wn, xn, 0, ul, false, false);
    };
    // loads past the last group reload it
    auto ldw = [&](int g) { return *reinterpret_cast<const uint4 *>(w + (int64_t)min(g, gl) * gs); };
    auto ldx = [&](int g) { return *reinterpret_cast<const uint4 *>(x + 8 * min(g, gl)); };
    uint4 wa[PF], xa[PF], wb[PF], xb[PF];
    auto load = [&](uint4 (&w4)[PF], uint4 (&x4)[PF], int g0) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            w4[p] = ldw(g0 + p);
            x4[p] = ldx(g0 + p);
        }
    };
    // the first group, then blocks of PF groups, double-buffered
    {
        const uint4 w0 = ldw(gf), x0 = ldx(gf);
        load(wa, xa, gf + 1);
        load(wb, xb, gf + 1 + PF);
        group(w0, x0, wa[0], xa[0], uf, gf < gl ? 8 : ul, true, k0 == 0);
    }
    auto run = [&](const uint4 (&w4)[PF], const uint4 (&x4)[PF], const uint4 (&wo)[PF], const uint4 (&xo)[PF],
                   int g0) __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            if (g0 + p > gl) break;
            body(w4[p], x4[p], p + 1 < PF ? w4[p + 1] : wo[0], p + 1 < PF ? x4[p + 1] : xo[0], g0 + p);
        }
    };
    for (int g0 = gf + 1; g0 <= gl; g0 += 2 * PF) {
        run(wa, xa, wb, xb, g0);
        if (g0 + PF > gl) break;
        load(wa, xa, g0 + 2 * PF);
        run(wb, xb, wa, xa, g0 + PF);
        load(wb, xb, g0 + 3 * PF);
    }
}

template <int MODE>
__device__ __forceinline__ void row_chain(const red16<MODE> &R, typename red16<MODE>::acc_t &acc, uint32_t &st,
                                          const uint16_t *__restrict__ w, int64_t gs, const uint16_t *x, int k0,
                                          int k1) {
    if constexpr (MODE == LNSHIP_SUM32) {
        row_chain_x32(R, acc, w, gs, x, k0, k1);
        return;
    }
    constexpr int PF = 4;
    const int ga = k0 >> 3, gl = (k1 - 1) >> 3;
    auto load = [&](uint4 (&b)[PF], int g0) {
#pragma unroll
        for (int p = 0; p < PF; p++) b[p] = *reinterpret_cast<const uint4 *>(w + (int64_t)min(g0 + p, gl) * gs);
    };
    auto run = [&](const uint4 (&b)[PF], int g0) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int g = g0 + p;
            if (g > gl) break;
            const uint4 xq = *reinterpret_cast<const uint4 *>(x + 8 * g);
            const uint32_t ww[4] = {b[p].x, b[p].y, b[p].z, b[p].w}, xx[4] = {xq.x, xq.y, xq.z, xq.w};
            // the products two at a time in 16-bit halves (xlns16_mul: the
            // log fields added, less the offset with unsigned saturation,
            // capped at 0x7fff; the signs xor'ed)
            uint32_t pl[4], ps[4];
#pragma unroll
            for (int i = 0; i < 4; i++) {
                pl[i] = pk_min_u16(pk_sub_sat_u16((ww[i] & 0x7fff7fffu) + (xx[i] & 0x7fff7fffu), 0x40004000u),
                                   0x7fff7fffu);
                ps[i] = ww[i] ^ xx[i];
            }
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int k = 8 * g + u;
                if (k < k0) continue;
                if (k >= k1) break;
                const uint32_t tl = (u & 1) ? pl[u >> 1] >> 16 : pl[u >> 1] & 0xffffu;
                const uint32_t ts = ((u & 1) ? ps[u >> 1] >> 16 : ps[u >> 1]) & k16_sign;
                if (k == 0) acc = R.start(ts | tl, st);
                else if constexpr (MODE == LNSHIP_SUM32)
                    R.add_lat(acc, tl << 16, ts << 16, [] {});
                else R.add_ls(acc, tl, ts, st);
            }
        }
    };
    if (k1 <= k0) return;
    uint4 wa[PF], wb[PF];
    load(wa, ga);
    for (int g0 = ga; g0 <= gl; g0 += 2 * PF) {
        load(wb, g0 + PF);
        run(wa, g0);
        if (g0 + PF > gl) break;
        load(wa, g0 + 2 * PF);
        run(wb, g0 + PF);
    }
}

// One workgroup per query head h (kv head h / rep): the kq scores (one chain
// of head_dim steps per cell), soft_max over them (k_softmax16's passes on one
// row), then the att outputs (one chain of n_kv steps per dim).  Between the
// nodes every value goes through F32 and back exactly as the separate nodes
// pass it on (the GEMV writes rev16 of its code, soft_max and the KQV GEMV
// convert their F32 inputs with cvt16), so the result is theirs bit for bit.
template <int MODE>
__global__ __launch_bounds__(k_block) void k_attn16(attn_args a, dev_tables T) {
    extern __shared__ __align__(16) char lds[];
    bool idle;
    // head hh = s nh + h: query head h of sequence s
    const int hh = attn_head(idle), sqn = hh / a.nh, h = hh - sqn * a.nh, kv = h / a.rep;
    if (idle) return;
    const red16<MODE> R = stage_for<MODE, true>(T, lds);
    const int hd = a.hd, n = a.n_kv, hp = (hd + 7) & ~7, rs = (n + 7) & ~7;
    uint16_t *xq = reinterpret_cast<uint16_t *>(lds + mm_xl_offset<MODE>());   // the query's codes
    uint16_t *c = xq + hp;                                                     // scores, then exps
    uint16_t *pc = c + rs;                                                     // KQV's activation codes
    __shared__ int32_t s_max;
    __shared__ uint32_t s_tot, s_tot2;   // the total (sum32: predicted, then the chain's)
    __shared__ float s_part[k_block / 64];
    __shared__ int s_last;
    __shared__ uint32_t s_vmax[k_attn_tail_hd];   // per dim: the largest V log past the last nonzero exp
    const bool tail_stop = hd <= k_attn_tail_hd;
    if (threadIdx.x == 0) {
        s_max = x16_canon(0xffffu);
        s_last = 0;
    }
    for (int d = threadIdx.x; d < k_attn_tail_hd; d += blockDim.x) s_vmax[d] = 0;
    if (a.qkv) {
        // (the position is one value for the whole workgroup)
        if (!attn_rope_store(a, T, h, kv, sqn, xq)) return;
    } else {
        for (int k = threadIdx.x; k < hp; k += blockDim.x)
            xq[k] = k < hd ? (uint16_t)x16_from_f32(T.cvt16, a.q[(int64_t)hh * hd + k]) : (uint16_t)0;
    }
    __syncthreads();
    // the scores, and soft_max's first pass over them
    const uint32_t sc = x16_from_f32(T.cvt16, a.scale);
    const bool has_mask = a.mask != nullptr;
    const uint16_t *kw = a.k + ((int64_t)sqn * a.nhkv + kv) * a.k_slice;
    const float *mrow = has_mask ? a.mask + (int64_t)sqn * n : nullptr;
    // Monte: each reduction starts where its node's would (kq: output
    // hh n + j of hd - 1 draws; soft_max: row hh of n - 1; kqv: output
    // hh hd + d of n - 1), from the node's own start
    uint32_t ms[3] = {0, 0, 0};
    if constexpr (MODE == LNSHIP_MONTE)
        for (int i = 0; i < 3; i++) ms[i] = monte_start(T, a.mseed[i], a.mstate, a.moff[i]);
    for (int j = threadIdx.x; j < n; j += blockDim.x) {
        uint32_t st = 0;
        if constexpr (MODE == LNSHIP_MONTE) st = lfsr_jump(T, ms[0], ((uint64_t)hh * n + j) * (uint64_t)(hd - 1));
        typename red16<MODE>::acc_t acc{};
        row_chain<MODE>(R, acc, st, kw + (int64_t)j * 8, a.k_gs, xq, 0, hd);
        const float mf = has_mask ? mrow[j] : 0.0f;
        // the score through F32 into xlns16 (the soft_max node reads it so)
        const uint32_t v = T.rho16[R.finish(acc) & 0xffffu], mk = x16_from_f32(T.cvt16, mf);
        const uint32_t vm = x16_mul(v, sc), va = x16_add_g(T.gauss16, vm, mk);
        const bool masked_out = has_mask && (mf <= -3.0e38f || mk == 0xffffu);
        const uint32_t w = v == 0xffffu || masked_out ? 0xffffu : (has_mask && (mk & k16_logmask)) ? va : vm;
        c[j] = (uint16_t)w;
        atomicMax(&s_max, x16_canon(w));
    }
    __syncthreads();
    {
        const int32_t cm = s_max;
        const uint32_t mx = (uint32_t)(uint16_t)(cm < 0 ? (cm ^ 0x7fff) : cm);
        for (int j = threadIdx.x; j < n; j += blockDim.x) {
            const uint32_t e = T.exp16[x16_add_g(T.gauss16, c[j], mx ^ k16_sign)];
            c[j] = (uint16_t)e;
            if (e & k16_logmask) atomicMax(&s_last, j);
        }
    }
    __syncthreads();
    const uint16_t *vw = a.v + ((int64_t)sqn * a.nhkv + kv) * a.v_slice;
    const int n_eff = s_last + 1;
    // the sum of exps up to the last nonzero one, as k_softmax16 runs it
    auto sum_chain = [&]() __attribute__((always_inline)) {
        uint32_t st = 0;
        if constexpr (MODE == LNSHIP_MONTE) st = lfsr_jump(T, ms[1], (uint64_t)hh * (uint64_t)(n - 1));
        typename red16<MODE>::acc_t acc = R.start(c[0], st);
        if (n_eff > 1) chain16<red16<MODE>, true>(R, acc, c, 1, n_eff, st);
        return R.finish(acc) & 0xffffu;
    };
    // threads t0, t0 + nt, ...: the largest V log of each dim over the cells
    // past the last nonzero exp
    auto tail_vmax = [&](int t0, int nt) __attribute__((always_inline)) {
        const int g0 = n_eff >> 3, ngt = ((n - 1) >> 3) - g0 + 1;
#pragma unroll 4
        for (int i = (int)threadIdx.x - t0; i < hd * ngt; i += nt) {
            const int d = i % hd, g = g0 + i / hd;
            const uint4 q4 = *reinterpret_cast<const uint4 *>(vw + (int64_t)d * 8 + (int64_t)g * a.v_gs);
            const uint32_t qq[4] = {q4.x, q4.y, q4.z, q4.w};
            uint32_t m = 0;
#pragma unroll
            for (int u = 0; u < 8; u++) {
                const int j = 8 * g + u;
                if (j >= n_eff && j < n) m = max(m, half16(qq[u >> 1], u & 1) & k16_logmask);
            }
            atomicMax(&s_vmax[d], m);
        }
    };
    // soft_max's output as KQV's mul_mat reads it: each probability through
    // F32 into xlns16
    auto stage_p = [&](uint32_t tot) __attribute__((always_inline)) {
        for (int j = threadIdx.x; j < rs; j += blockDim.x)
            pc[j] = j < n ? (uint16_t)T.rho16[x16_div(c[j], tot)] : (uint16_t)0;
    };
    // The att output of dim d.  Past the last nonzero exp every p has one
    // code (all those exps are 0), so a product there has the log
    // clamp(v + p - 0x4000) and the largest is that of the largest V log.  A
    // lane's chain stops at the last nonzero exp when that largest product
    // lies at or beyond the adder's essential zero below its sum: every
    // later term would add nothing (and keep the sum's sign)
    auto out_chain = [&](int d) __attribute__((always_inline)) {
        const uint32_t p_tail = n_eff < n ? pc[n_eff] & k16_logmask : 0u;
        const uint16_t *vr = vw + (int64_t)d * 8;
        uint32_t st = 0;
        if constexpr (MODE == LNSHIP_MONTE) st = lfsr_jump(T, ms[2], ((uint64_t)hh * hd + d) * (uint64_t)(n - 1));
        typename red16<MODE>::acc_t acc{};
        bool rest = n_eff < n;
        if (rest && tail_stop) {
            row_chain<MODE>(R, acc, st, vr, a.v_gs, pc, 0, n_eff);
            const uint32_t tmax = (uint32_t)min(max((int32_t)(s_vmax[d] + p_tail) - (int32_t)k16_one, 0),
                                                (int32_t)k16_logmask);
            if constexpr (MODE == LNSHIP_BASE) rest = acc.l < tmax + (uint32_t)k16_esszer + 1u;
            // Monte: no draw moves a sum at a distance of k16_mc_end or more
            else if constexpr (MODE == LNSHIP_MONTE) rest = acc.l < tmax + (uint32_t)k16_mc_end;
            else rest = acc.l < (tmax << 16) + k32_esszer;   // xlns32 accumulators (sum32, lpvip)
            if (rest) row_chain<MODE>(R, acc, st, vr, a.v_gs, pc, n_eff, n);
        } else {
            row_chain<MODE>(R, acc, st, vr, a.v_gs, pc, 0, n);
        }
        return R.finish(acc) & 0xffffu;
    };
    // sum32, with a wave beside the output chains' (head_dim <= 192): the
    // output chains start at once from a predicted total while that wave's
    // first lane runs the sum's chain, and run again when the total differs.
    // The prediction sums the exps' values in F32 and rounds the log to the
    // nearest xlns16 step, which is the chain's narrowed xlns32 sum unless
    // that sum lies within the chain's error (and the F32 sum's) of a
    // rounding boundary.
    const int sum_lane = (hd + 63) & ~63;
    if (MODE == LNSHIP_SUM32 && sum_lane < (int)blockDim.x) {
        float part = 0.0f;
        for (int j = threadIdx.x; j < n_eff; j += blockDim.x)
            part += exp2f((float)((int)(c[j] & k16_logmask) - (int)k16_one) * (1.0f / 128.0f));
        for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o);
        if ((threadIdx.x & 63) == 0) s_part[threadIdx.x >> 6] = part;
        if (tail_stop && n_eff < n) tail_vmax(0, (int)blockDim.x);
        __syncthreads();
        if (threadIdx.x == 0) {
            float S = 0.0f;
            for (int i = 0; i < k_block / 64; i++) S += s_part[i];
            const float l = S > 0.0f ? floorf(log2f(S) * 128.0f + 0.5f) + (float)k16_one : 0.0f;
            s_tot = ((uint32_t)fminf(fmaxf(l, 0.0f), (float)k16_logmask) + a.skew) & 0xffffu;
        }
        __syncthreads();
        const uint32_t tot = s_tot;
        stage_p(tot);
        __syncthreads();
        uint32_t res = 0;
        if ((int)threadIdx.x < hd) res = out_chain((int)threadIdx.x);
        else if ((int)threadIdx.x == sum_lane) s_tot2 = sum_chain();
        __syncthreads();
        // (every thread reads the same word after the barrier)
        if (s_tot2 != tot) {
            stage_p(s_tot2);
            __syncthreads();
            if ((int)threadIdx.x < hd) res = out_chain((int)threadIdx.x);
        }
        if ((int)threadIdx.x < hd) a.dst[(int64_t)hh * hd + threadIdx.x] = T.rev16[res];
        return;
    }
    if (threadIdx.x < 64u) {
        // on every lane of the first wave (as the row sums of k_rms16)
        const uint32_t t = sum_chain();
        if (threadIdx.x == 0) s_tot = t;
    } else if (tail_stop && n_eff < n) {
        // meanwhile, on the other waves: the tail's V maxima
        tail_vmax(64, (int)blockDim.x - 64);
    }
    __syncthreads();
    stage_p(s_tot);
    __syncthreads();
    for (int d = threadIdx.x; d < hd; d += blockDim.x) a.dst[(int64_t)hh * hd + d] = T.rev16[out_chain(d)];
}

// ---- LNS32 decode attention: KQ, soft_max and KQV of one token in one launch --
// row_chain_x32 over xlns32 codes (the LNS32 GEMV's terms: 4-byte weights and
// activations, a group of eight 32 bytes; x32_mul products, as k_mm32's
// single-chain loop forms them, each in the first round trip of the step
// before it)
__device__ __forceinline__ void row_chain32(const x32_tab &O, acc_ls &acc, const uint32_t *__restrict__ w,
                                            int64_t gs, const uint32_t *x, int k0, int k1) {
    if (k1 <= k0) return;
    constexpr int PF = 2;
    const int gl = (k1 - 1) >> 3;
    auto term_at = [&](int k) { return x32_mul(w[(int64_t)(k >> 3) * gs + (k & 7)], x[k]); };
    // term 0 starts the sum; the steps add terms ks .. k1 - 1
    const int ks = k0 == 0 ? 1 : k0;
    if (k0 == 0) {
        const uint32_t t0 = term_at(0);
        acc = {t0 & k32_logmask, t0 & k32_sign};
        if (k1 == 1) return;
    }
    uint32_t t = term_at(ks);
    uint32_t uf = acc.s ^ (t & k32_sign);
    struct g8 {
        uint4 lo, hi;
    };
    // steps [u0, u1) of group g; the groups strictly inside the row run all
    // eight with no bounds test
    auto group = [&](const g8 &wq, const g8 &xq, const g8 &wn, const g8 &xn, int u0, int u1)
                     __attribute__((always_inline)) {
        const uint32_t ww[8] = {wq.lo.x, wq.lo.y, wq.lo.z, wq.lo.w, wq.hi.x, wq.hi.y, wq.hi.z, wq.hi.w};
        const uint32_t xx[8] = {xq.lo.x, xq.lo.y, xq.lo.z, xq.lo.w, xq.hi.x, xq.hi.y, xq.hi.z, xq.hi.w};
#pragma unroll
        for (int u = 0; u < 8; u++) {
            if (u < u0 || u >= u1) continue;
            uint32_t tn = 0;
            auto next = [&] {
                tn = u < 7 ? x32_mul(ww[u + 1], xx[u + 1]) : x32_mul(wn.lo.x, xn.lo.x);
                return tn & k32_sign;
            };
            uf = x32_add_step(O, acc, t & k32_logmask, t & k32_sign, uf, next, [] {});
            t = tn;
        }
    };
    const int g1 = ks >> 3, ul = k1 - 8 * gl;
    auto body = [&](const g8 &wq, const g8 &xq, const g8 &wn, const g8 &xn, int g) __attribute__((always_inline)) {
        if (g > g1 && g < gl) group(wq, xq, wn, xn, 0, 8);
        else group(wq, xq, wn, xn, g == g1 ? ks & 7 : 0, g == gl ? ul : 8);
    };
    // blocks of PF groups, double-buffered; loads past the last group reload it
    g8 wa[PF], xa[PF], wb[PF], xb[PF];
    auto load = [&](g8 (&w4)[PF], g8 (&x4)[PF], int g0) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            const int g = min(g0 + p, gl);
            const uint4 *wp = reinterpret_cast<const uint4 *>(w + (int64_t)g * gs);
            const uint4 *xp = reinterpret_cast<const uint4 *>(x + 8 * g);
            w4[p] = {wp[0], wp[1]};
            x4[p] = {xp[0], xp[1]};
        }
    };
    auto run = [&](const g8 (&w4)[PF], const g8 (&x4)[PF], const g8 (&wo)[PF], const g8 (&xo)[PF], int g0)
                   __attribute__((always_inline)) {
#pragma unroll
        for (int p = 0; p < PF; p++) {
            if (g0 + p > gl) break;
            body(w4[p], x4[p], p + 1 < PF ? w4[p + 1] : wo[0], p + 1 < PF ? x4[p + 1] : xo[0], g0 + p);
        }
    };
    load(wa, xa, g1);
    load(wb, xb, g1 + PF);
    for (int g0 = g1; g0 <= gl; g0 += 2 * PF) {
        run(wa, xa, wb, xb, g0);
        if (g0 + PF > gl) break;
        load(wa, xa, g0 + 2 * PF);
        run(wb, xb, wa, xa, g0 + PF);
        load(wb, xb, g0 + 3 * PF);
    }
}

// one xlns32 addition as the single-chain step makes it (the tables of
// stage_for<SUM32, true>), for the element passes of a kernel that stages
// that image
__device__ __forceinline__ uint32_t x32_add_dec(const x32_tab &O, uint32_t x, uint32_t y) {
    acc_ls c{x & k32_logmask, x & k32_sign};
    const uint32_t ys = y & k32_sign;
    x32_add_step(O, c, y & k32_logmask, ys, c.s ^ ys, [] { return 0u; }, [] {});
    return c.s | c.l;
}

struct attn32_args {
    const float *q;
    const uint32_t *k, *v;
    int64_t k_gs, k_slice, v_gs, v_slice;   // codes between groups of eight; between kv heads
    const float *mask;
    float scale;
    float *dst;
    int hd, n_kv, rep;   // head_dim, cells, query heads per kv head
};

// The LNS32 backend's decode attention as k_attn16 runs the LNS16 one: one
// workgroup per query head h (kv head h / rep), the kq scores (one chain of
// head_dim steps per cell), k_softmax32's passes and sum over them, then the
// att outputs (one chain of n_kv steps per dim).  Between the nodes every
// value takes the F32 round trip the separate nodes pass it on (the GEMV
// writes x32_to_f32 of its code, soft_max and the KQV GEMV convert their F32
// inputs with x32_from_f32), so the result is theirs bit for bit.  The
// soft_max total is an xlns32 code, far finer than its chain's error, so the
// KQV chains wait for it (no predicted start as in sum32).
__global__ __launch_bounds__(k_block) void k_attn32(attn32_args a, dev_tables T) {
    extern __shared__ __align__(16) char lds[];
    bool idle;
    const int h = attn_head(idle), kv = h / a.rep;
    if (idle) return;
    const red16<LNSHIP_SUM32> R = stage_for<LNSHIP_SUM32, true>(T, lds);
    const int hd = a.hd, n = a.n_kv, hp = (hd + 7) & ~7, rs = (n + 7) & ~7;
    uint32_t *xq = reinterpret_cast<uint32_t *>(lds + k_lds_tab32);   // the query's codes
    uint32_t *c = xq + hp;                                             // scores, then exps
    uint32_t *pc = c + rs;                                             // KQV's activation codes
    __shared__ int32_t s_max;
    __shared__ uint32_t s_tot;
    __shared__ int s_last;
    if (threadIdx.x == 0) {
        s_max = x32_canon(0xffffffffu);
        s_last = 0;
    }
    for (int k = threadIdx.x; k < hp; k += blockDim.x) xq[k] = k < hd ? x32_from_f32(a.q[(int64_t)h * hd + k]) : 0u;
    __syncthreads();
    // the scores, and soft_max's first pass over them (k_softmax32's)
    const uint32_t sc = x32_from_f32(a.scale);
    const uint32_t *kw = a.k + kv * a.k_slice;
    for (int j = threadIdx.x; j < n; j += blockDim.x) {
        acc_ls acc{};
        row_chain32(R.O, acc, kw + (int64_t)j * 8, a.k_gs, xq, 0, hd);
        uint32_t v = x32_from_f32(x32_to_f32(acc.s | acc.l));
        if (v != 0xffffffffu) {
            v = x32_mul(v, sc);
            if (a.mask) {
                const float mf = a.mask[j];
                const uint32_t mk = mf <= -3.0e38f ? 0xffffffffu : x32_from_f32(mf);
                if (mk == 0xffffffffu) v = 0xffffffffu;
                else if (mk & k32_logmask) v = x32_add_dec(R.O, v, mk);
            }
        }
        c[j] = v;
        atomicMax(&s_max, x32_canon(v));
    }
    __syncthreads();
    {
        const int32_t cm = s_max;
        const uint32_t mx = (uint32_t)(cm < 0 ? (cm ^ 0x7fffffff) : cm);
        for (int j = threadIdx.x; j < n; j += blockDim.x) {
            const float fv = x32_to_f32(x32_add_dec(R.O, c[j], mx ^ k32_sign));
            const uint32_t e = x32_from_f32((float)exp((double)fv));
            c[j] = e;
            if (e & k32_logmask) atomicMax(&s_last, j);
        }
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        // the sum of exps up to the last nonzero one, as k_softmax32 runs it
        acc_ls acc{c[0] & k32_logmask, c[0] & k32_sign};
        const int n_eff = s_last + 1;
        if (n_eff > 1) chain32<true>(R.O, acc, c, 1, n_eff);
        s_tot = acc.s | acc.l;
    }
    __syncthreads();
    // soft_max's output as KQV's mul_mat reads it: each probability through
    // F32 into xlns32
    const uint32_t tot = s_tot;
    for (int j = threadIdx.x; j < rs; j += blockDim.x)
        pc[j] = j < n ? x32_from_f32(x32_to_f32(x32_div(c[j], tot))) : 0u;
    __syncthreads();
    const uint32_t *vw = a.v + kv * a.v_slice;
    for (int d = threadIdx.x; d < hd; d += blockDim.x) {
        acc_ls acc{};
        row_chain32(R.O, acc, vw + (int64_t)d * 8, a.v_gs, pc, 0, n);
        a.dst[(int64_t)h * hd + d] = x32_to_f32(acc.s | acc.l);
    }
}

__global__ __launch_bounds__(k_block) void k_softmax32(sm_args a, dev_tables T) {
    extern __shared__ __align__(16) char lds[];
    const red16<LNSHIP_SUM32> R = stage_tables<LNSHIP_SUM32>(T, lds);
    uint32_t *c = reinterpret_cast<uint32_t *>(lds + k_lds_tab32);
    __shared__ int32_t s_max[64];
    __shared__ uint32_t s_tot[64];
    __shared__ const float *s_mrow[64];
    __shared__ int s_last[64];   // a row's last element with a nonzero exp
    const int64_t r0 = (int64_t)blockIdx.x * a.rb;
    const int nr = (int)min<int64_t>(a.rb, a.ne1 * a.ne2 * a.ne3 - r0);
    const int64_t ne = (int64_t)nr * a.n;
    const int n = (int)a.n, nel = nr * n;
    const int rs = ((int)a.n + 3) & ~3;   // LDS rows 16-byte aligned
    if ((int)threadIdx.x < nr) {
        s_last[threadIdx.x] = 0;
        s_max[threadIdx.x] = x32_canon(0xffffffffu);
        s_mrow[threadIdx.x] = a.mask ? mask_row(a, r0 + threadIdx.x) : nullptr;
    }
    __syncthreads();
    const uint32_t sc = x32_from_f32(a.scale);
    // loads in batches of B per thread (past the end the last element again:
    // the same value to the same place)
    constexpr int B = 8;
    const int nt = (int)blockDim.x;
    for (int e0 = threadIdx.x; e0 < nel; e0 += B * nt) {
        float f[B], mf[B];
#pragma unroll
        for (int q = 0; q < B; q++) {
            const int e = min(e0 + q * nt, nel - 1), r = e / n, i = e - r * n;
            f[q] = a.src[(r0 + r) * a.n + i];
            mf[q] = a.mask ? s_mrow[r][i] : 0.0f;
        }
#pragma unroll
        for (int q = 0; q < B; q++) {
            const int e = min(e0 + q * nt, nel - 1), r = e / n;
            uint32_t v = x32_from_f32(f[q]);
            if (v != 0xffffffffu) {
                v = x32_mul(v, sc);
                if (a.mask) {
                    const uint32_t mk = mf[q] <= -3.0e38f ? 0xffffffffu : x32_from_f32(mf[q]);
                    if (mk == 0xffffffffu) v = 0xffffffffu;
                    else if (mk & k32_logmask) v = x32_add_lds(R.O, v, mk);
                }
            }
            c[e + r * (rs - n)] = v;
            atomicMax(&s_max[r], x32_canon(v));
        }
    }
    __syncthreads();
    for (int64_t e = threadIdx.x; e < ne; e += blockDim.x) {
        const int r = (int)(e / a.n);
        const int32_t cm = s_max[r];
        const uint32_t mx = (uint32_t)(cm < 0 ? (cm ^ 0x7fffffff) : cm);
        const int64_t o = e + r * (rs - a.n);
        const float fv = x32_to_f32(x32_add_lds(R.O, c[o], mx ^ k32_sign));
        c[o] = x32_from_f32((float)exp((double)fv));
        if (c[o] & k32_logmask) atomicMax(&s_last[r], (int)(e - (int64_t)r * a.n));
    }
    __syncthreads();
    // (all 64 lanes, as in k_rms16)
    if (threadIdx.x < 64u) {
        const int r = min((int)threadIdx.x, nr - 1);
        const uint32_t *row = c + r * rs;
        acc_ls acc{row[0] & k32_logmask, row[0] & k32_sign};
        // trailing exps of log 0 add nothing to a sum of at least 1 (as in
        // k_softmax16): the chain stops at the last nonzero exp
        const int n_eff = s_last[r] + 1;
        if (n_eff > 1) chain32<true>(R.O, acc, row, 1, n_eff);   // exps: positive
        if ((int)threadIdx.x < nr) s_tot[r] = acc.s | acc.l;
    }
    __syncthreads();
    for (int64_t e = threadIdx.x; e < ne; e += blockDim.x) {
        const int r = (int)(e / a.n);
        a.dst[r0 * a.n + e] = x32_to_f32(x32_div(c[e + r * (rs - a.n)], s_tot[r]));
    }
}

// ---- data movement of a device-resident ggml graph (no LNS arithmetic) ----
// Element types: 0 F32, 1 F16 (IEEE half; F32 -> F16 rounds to nearest even).

__device__ __forceinline__ int64_t view_offset(const strided4 &g, int64_t i) {
    const int64_t i0 = i % g.ne[0];
    i /= g.ne[0];
    const int64_t i1 = i % g.ne[1];
    i /= g.ne[1];
    const int64_t i2 = i % g.ne[2], i3 = i / g.ne[2];
    return i0 * g.nb[0] + i1 * g.nb[1] + i2 * g.nb[2] + i3 * g.nb[3];
}

template <int TY>
__device__ __forceinline__ float load_elem(const char *p) {
    return TY ? __half2float(*reinterpret_cast<const __half *>(p)) : *reinterpret_cast<const float *>(p);
}
template <int TY>
__device__ __forceinline__ void store_elem(char *p, float v) {
    if (TY) *reinterpret_cast<__half *>(p) = __float2half_rn(v);
    else *reinterpret_cast<float *>(p) = v;
}

// element i of src (in its logical order) -> element i of dst
template <int ST, int DT>
__global__ void k_copy(const char *__restrict__ src, strided4 gs, char *__restrict__ dst, strided4 gd) {
    const int64_t n = gs.ne[0] * gs.ne[1] * gs.ne[2] * gs.ne[3];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x)
        store_elem<DT>(dst + view_offset(gd, i), load_elem<ST>(src + view_offset(gs, i)));
}

// ids: ne[0..2], nb[0..2] of the index tensor
struct ids3 {
    int64_t ne[3];
    int64_t nb[3];
};

__device__ __forceinline__ int64_t load_id(const char *ids, const ids3 &g, int64_t i0, int64_t i1, int64_t i2,
                                           int i64) {
    const char *p = ids + i0 * g.nb[0] + i1 * g.nb[1] + i2 * g.nb[2];
    return i64 ? *reinterpret_cast<const int64_t *>(p) : (int64_t)*reinterpret_cast<const int32_t *>(p);
}

// dst row (i10, i11, i12) = src row ids[i10, i11, i12] of src slice (i11, i12)
template <int ST>
__global__ void k_get_rows(const char *__restrict__ src, strided4 gs, const char *__restrict__ ids, ids3 gi,
                           float *__restrict__ dst, strided4 gd, unsigned long long *err) {
    const int64_t nc = gs.ne[0], nr = gi.ne[0] * gi.ne[1] * gi.ne[2];
    const int64_t n = nc * nr;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        const int64_t c = i % nc, r = i / nc;
        const int64_t i10 = r % gi.ne[0], t = r / gi.ne[0];
        const int64_t i11 = t % gi.ne[1], i12 = t / gi.ne[1];
        const int64_t row = load_id(ids, gi, i10, i11, i12, 0);
        if (row < 0 || row >= gs.ne[1]) {
            index_fault(err, row);
            continue;
        }
        const float v = load_elem<ST>(src + c * gs.nb[0] + row * gs.nb[1] + i11 * gs.nb[2] + i12 * gs.nb[3]);
        *reinterpret_cast<float *>(reinterpret_cast<char *>(dst) + c * gd.nb[0] + i10 * gd.nb[1] + i11 * gd.nb[2] +
                                   i12 * gd.nb[3]) = v;
    }
}

// dst row ids[r, i02 % ne11, i03 % ne12] of dst slice (i02, i03) = src row
// (r, i02, i03), converted to the destination type
template <int DT>
__global__ void k_set_rows(const char *__restrict__ src, strided4 gs, const char *__restrict__ ids, ids3 gi,
                           int ids_i64, char *__restrict__ dst, strided4 gd, unsigned long long *err) {
    const int64_t nc = gs.ne[0];
    const int64_t n = nc * gs.ne[1] * gs.ne[2] * gs.ne[3];
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        const int64_t c = i % nc, t0 = i / nc;
        const int64_t r = t0 % gs.ne[1], t1 = t0 / gs.ne[1];
        const int64_t i02 = t1 % gs.ne[2], i03 = t1 / gs.ne[2];
        const int64_t row = load_id(ids, gi, r, i02 % gi.ne[1], i03 % gi.ne[2], ids_i64);
        if (row < 0 || row >= gd.ne[1]) {
            index_fault(err, row);
            continue;
        }
        const float v = load_elem<0>(src + c * gs.nb[0] + r * gs.nb[1] + i02 * gs.nb[2] + i03 * gs.nb[3]);
        store_elem<DT>(dst + c * gd.nb[0] + row * gd.nb[1] + i02 * gd.nb[2] + i03 * gd.nb[3], v);
    }
}

// lpvip's db at d0 .. d0 + n - 1 (a test hook: the db function is checked
// over its whole exact-branch domain against the host)
__global__ void k_lpvip_db_range(uint32_t d0, uint32_t n, int32_t *__restrict__ out, const double *lp) {
    for (uint32_t i = blockIdx.x * blockDim.x + threadIdx.x; i < n; i += blockDim.x * gridDim.x)
        out[i] = lpvip_db(lp, d0 + i);
}

// The xlns32 adder over its LDS tables on code pairs, in the form the kernels
// run it: FORM 0 the multi-chain step, 1 the single-chain step of the decode
// GEMVs, 2 the positive-sum step (sign bits ignored), 3 the positive-sum step
// over the pair image (sign bits ignored).
template <int FORM>
__global__ __launch_bounds__(k_block) void k_x32_add_lds(const uint32_t *__restrict__ x, const uint32_t *__restrict__ y,
                                                         uint32_t *__restrict__ out, int64_t n, dev_tables T) {
    extern __shared__ __align__(16) char lds[];
    red16<LNSHIP_SUM32> R{};
    pos_tab P{};
    if constexpr (FORM == 3) P = stage_pos32(T, lds);
    else R = stage_for<LNSHIP_SUM32, FORM == 1>(T, lds);
    __syncthreads();
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        const uint32_t a = x[i], b = y[i];
        uint32_t r;
        if constexpr (FORM == 0) {
            r = x32_add_lds(R.O, a, b);
        } else if constexpr (FORM == 1) {
            acc_ls c{a & k32_logmask, a & k32_sign};
            const uint32_t ts = b & k32_sign;
            x32_add_step(R.O, c, b & k32_logmask, ts, c.s ^ ts, [] { return 0u; }, [] {});
            r = c.s | c.l;
        } else if constexpr (FORM == 2) {
            r = x32_add_pos(R.O, a & k32_logmask, b & k32_logmask);
        } else {
            r = x32_add_pos2(P, a & k32_logmask, b & k32_logmask);
        }
        out[i] = r;
    }
}

__global__ void k_causal_mask(const int32_t *__restrict__ pos, int64_t ntok, int64_t n_kv, float *__restrict__ mask) {
    const int64_t n = ntok * n_kv;
    for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)blockDim.x * gridDim.x) {
        const int64_t t = i / n_kv, j = i - t * n_kv;
        mask[i] = j <= pos[t] ? 0.0f : -INFINITY;
    }
}

// ---- host helpers -------------------------------------------------------------

// rows beside tab_bytes of LDS tables, staged at a 16-byte stride
static int64_t max_row(int tab_bytes, int elem_bytes) {
    return ((k_lds_bytes - ((tab_bytes + 15) & ~15) - k_lds_static) / 16) * (16 / elem_bytes);
}

// Rows per workgroup of a row kernel: one chain lane per row, so a block
// takes as long as one chain plus its element passes over all its rows.
// The most rows LDS holds decide how many rounds of blocks the GPU needs;
// within that many rounds the rows are spread over every block slot, so that
// no block carries more rows (longer element passes) than it must.
static int rows_per_block(int tab_bytes, int64_t ncols, int elem_bytes, int64_t nrows, int cus) {
    const int64_t tabs = (tab_bytes + 15) & ~15;
    const int64_t row = std::max<int64_t>(1, ncols * elem_bytes);
    const int64_t rb_max = std::min<int64_t>(64, (k_lds_bytes - tabs - k_lds_static) / row);
    if (rb_max < 1 || nrows < 1) return (int)rb_max;
    const int64_t slots = (int64_t)std::max(cus, 1) * std::max<int64_t>(1, k_lds_bytes / (tabs + rb_max * row));
    const int64_t rounds = (nrows + rb_max * slots - 1) / (rb_max * slots);
    return (int)std::min<int64_t>(rb_max, (nrows + rounds * slots - 1) / (rounds * slots));
}

template <class K>
static int set_lds(K kernel, int bytes) {
    LNSHIP_HIP(hipFuncSetAttribute((const void *)kernel, hipFuncAttributeMaxDynamicSharedMemorySize, bytes));
    return 0;
}

static int pack_common(int w32, const void *src, int src_is_f16, int64_t src_ld, int64_t src_slice, void *dst,
                       int64_t K, int64_t M, int64_t nslices, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (K < 0 || M < 0 || nslices < 0 || src_ld < K || nslices > 65535)
        return fail(LNSHIP_EINVAL, "pack: bad shape%s");
    if (src_is_f16 < 0 || src_is_f16 > (w32 ? 1 : 2)) return fail(LNSHIP_EINVAL, "pack: bad source type%s");
    if (K == 0 || M == 0 || nslices == 0) return 0;
    const int64_t kp = (K + 7) & ~(int64_t)7;
    dim3 grid(grid_for(M * kp, 2), (unsigned)nslices);
    if (w32)
        hipLaunchKernelGGL(k_pack<1>, grid, dim3(k_block), 0, (hipStream_t)stream, src, src_is_f16, src_ld, src_slice,
                           dst, M, K, kp, s->T.cvt16);
    else
        hipLaunchKernelGGL(k_pack<0>, grid, dim3(k_block), 0, (hipStream_t)stream, src, src_is_f16, src_ld, src_slice,
                           dst, M, K, kp, s->T.cvt16);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

static int check_mm(const lnship_mul_mat_args *a) {
    if (!a || a->K < 0 || a->M < 0 || a->N < 0 || a->ne02 <= 0 || a->ne03 <= 0 || a->ne12 <= 0 || a->ne13 <= 0)
        return fail(LNSHIP_EINVAL, "mul_mat: bad shape%s");
    if (a->ne12 % a->ne02 || a->ne13 % a->ne03) return fail(LNSHIP_EINVAL, "mul_mat: slices do not broadcast%s");
    if (a->ne12 * a->ne13 > 65535) return fail(LNSHIP_ERANGE, "mul_mat: more than 65535 activation slices%s");
    const int64_t xld = a->x_ld ? a->x_ld : a->K;
    if (xld < a->K) return fail(LNSHIP_EINVAL, "mul_mat: x_ld < K%s");
    if (a->w_mstride && a->w_mstride < a->M) return fail(LNSHIP_EINVAL, "mul_mat: w_mstride < M%s");
    if (a->dst_ld && a->dst_ld < a->M) return fail(LNSHIP_EINVAL, "mul_mat: dst_ld < M%s");
    return 0;
}

static int64_t mm16_tables_bytes(int mode) {
    switch (mode) {
        case LNSHIP_BASE: return mm_xl_offset<LNSHIP_BASE>();
        case LNSHIP_MONTE: return mm_xl_offset<LNSHIP_MONTE>();
        case LNSHIP_LPVIP: return mm_xl_offset<LNSHIP_LPVIP>();
        default: return mm_xl_offset<LNSHIP_SUM32>();
    }
}

// whether `cols` activation rows of kp codes fit in LDS next to the tables
static bool mm16_xl(int mode, int cols, int64_t kp) {
    return mm16_tables_bytes(mode) + (int64_t)cols * kp * 2 + k_xl_pad <= k_lds_bytes - 1024;
}

// Columns per lane.  Every output is a K-long dependent chain, so a lane is
// fastest with one chain; the fewest columns per lane whose workgroups all
// fit on the GPU at once (LDS and about three waves per SIMD allowing) wins.
// When even eight columns per lane take more than one round, throughput
// decides: eight columns share one weight load and one decode per step.
static int mm16_nc(int mode, int64_t M, int64_t N, int64_t nslices, int64_t kp, int cus) {
    const int64_t wg_m = (M + k_block - 1) / k_block;
    for (int nc : {1, 4, 8}) {
        const int64_t lds = mm16_tables_bytes(mode) + (mm16_xl(mode, nc, kp) ? (int64_t)nc * kp * 2 : 0);
        const int64_t per_cu = std::max<int64_t>(1, std::min<int64_t>(3, k_lds_bytes / std::max<int64_t>(lds, 1)));
        if (wg_m * ((N + nc - 1) / nc) * nslices <= (int64_t)std::max(cus, 1) * per_cu) return nc;
    }
    return 8;
}

struct mm16_shape {
    int nc, cg;   // columns per lane, column groups per workgroup
    bool xl;      // activations converted into LDS inside the kernel
};

// The xlns32 tables leave room for one workgroup per CU, so the sum32 and
// xlns32 GEMVs take their waves per SIMD from column groups.  Time per k of a
// shape is rounds x (chains per SIMD) x (time per chain step at that many
// waves per SIMD); measured on MI355X, a chain step costs 166 ns with one
// wave and one chain (the adder's latency), 148 ns with one wave of several
// chains, 103 ns at two waves and 85 ns at four (the VALU issue rate of 49
// instructions).
static mm16_shape mm_shape_x32(int64_t M, int64_t N, int64_t nslices, int64_t kp, int cus, int max_nc) {
    // (one wave of several chains, or two waves of two or more, never wins)
    static const int shapes[][2] = {{1, 1}, {1, 2}, {1, 4}, {2, 4}, {4, 4}, {8, 4}};
    const int64_t wg_m = (M + k_block - 1) / k_block;
    mm16_shape best{1, 1, mm16_xl(LNSHIP_SUM32, 1, kp)};
    int64_t best_cost = -1;
    for (const auto &sh : shapes) {
        const int nc = sh[0], cg = sh[1];
        if ((nc * cg > 1 && nc * cg > N) || nc > max_nc) continue;
        const int64_t wgs = wg_m * ((N + nc * cg - 1) / (nc * cg)) * nslices;
        const int64_t rounds = (wgs + std::max(cus, 1) - 1) / std::max(cus, 1);
        const int64_t step = cg == 1 ? (nc == 1 ? 166 : 148) : cg == 2 ? 103 : 85;
        const int64_t cost = rounds * cg * nc * step;
        // ties go to more columns per workgroup (one weight decode serves them)
        if (best_cost < 0 || cost <= best_cost) {
            best = {nc, cg, mm16_xl(LNSHIP_SUM32, nc * cg, kp)};
            best_cost = cost;
        }
    }
    return best;
}

// Workgroups of a launch are dealt round-robin to the XCDs (eight on MI355X,
// each with its own L2).  A sum32 GEMV workgroup first stages the 130 KB
// xlns32 image into LDS (one workgroup per CU at that size); in a launch of
// few workgroups each lands on another XCD and misses the image in that
// XCD's L2.  Launched 2^sh times wider, with only the workgroups whose index
// is a multiple of 2^sh working, the working ones fall on 8 >> sh XCDs and
// share those L2s' copies.  sh is the largest (at most 3) for which those
// XCDs still hold every working workgroup at one per CU.
// Rows per wave of the single-chain GEMVs: 16, or 0 for 64-row waves;
// lnship_test_decode_width sets it
static int g_decode_w = 16;

// 16-row waves for a launch of `chains` chains (rows x columns x slices,
// one column per workgroup column) while they fill at most one wave slot per
// SIMD: the chains are bound by their dependent steps, and a step with only
// the first 16 lanes of its wave active is shorter
static bool narrow_mm(int64_t chains, int cus) { return g_decode_w == 16 && chains <= (int64_t)cus * 4 * 16; }
// rows per wave of a single-chain GEMV outside sum32 (its chains on all 64
// lanes): fewer chains per wave branch apart less often, while the launch
// still fits one wave per SIMD (two waves on a SIMD cost more: lpvip up|gate
// of 8 columns, 24576 chains: 170.6 us on 64-row waves, 161.9 on 32, 190.1
// on 16 at two per SIMD); lpvip narrows further than 16; 0: 64-row waves
static int narrow_w(int mode, int64_t chains, int cus) {
    if (g_decode_w != 16) return 0;
    const int64_t slots = (int64_t)cus * 4;
    if (mode == LNSHIP_LPVIP && chains <= slots * 4) return 4;
    if (mode == LNSHIP_LPVIP && chains <= slots * 8) return 8;
    return chains <= slots * 16 ? 16 : chains <= slots * 32 ? 32 : 0;
}

// the grid of nh attention heads placed by attn_head: every block up to the
// last head's, the multiples of 8 idle
static unsigned attn_grid(int64_t nh) { return (unsigned)(nh + 1 + (nh - 1) / 7); }

static uint32_t xcd_shift(uint64_t wgs, int cus) {
    const uint64_t per_xcd = (uint64_t)std::max(cus / 8, 1);
    uint32_t sh = 3;
    while (sh > 0 && wgs > (per_xcd << (3 - sh))) sh--;
    return sh;
}

static mm16_shape mm16_choose(int mode, int64_t M, int64_t N, int64_t nslices, int64_t kp, int cus) {
    if (mode == LNSHIP_SUM32) return mm_shape_x32(M, N, nslices, kp, cus, 8);
    const int nc = mm16_nc(mode, M, N, nslices, kp, cus);
    return {nc, 1, mm16_xl(mode, nc, kp)};
}

template <int MODE, int NC, bool XL, int CG, int W = 64>
static int launch_mm16(const mm_args16 &m, const dev_tables &T, int64_t nslices, int cus, hipStream_t st) {
    // prefetch depth within 128 VGPRs at four waves per SIMD
    constexpr int PF = NC == 1 ? (CG >= 4 ? 4 : 8) : NC == 2 ? 2 : (NC == 4 && CG < 4) ? 2 : 1;
    const int lds = mm_xl_offset<MODE>() + (XL ? (int)(NC * CG * m.kp * 2) + k_xl_pad : 0);
    static_assert(PF * 16 <= k_xl_pad, "prefetch past the activation rows stays in the padding");
    // weight offsets within a block of PF groups are 32-bit
    if ((uint64_t)m.w_mstride * 16 * PF + (uint64_t)m.M * 16 > 0xffffffffu)
        return fail(LNSHIP_ERANGE, "mul_mat: weight rows too long for 32-bit block offsets%s");
    if (lds > 64 * 1024)
        if (int rc = set_lds(k_mm16<MODE, NC, PF, XL, CG, W>, lds)) return rc;
    constexpr int rows = W < 64 ? k_block / 64 * W : k_block;   // rows per workgroup
    dim3 grid((unsigned)((m.M + rows - 1) / rows), (unsigned)((m.N + NC * CG - 1) / (NC * CG)), (unsigned)nslices);
    if (grid.x > 2147483647u || grid.y > 65535u) return fail(LNSHIP_ERANGE, "mul_mat: grid too large%s");
    mm_args16 mx = m;
    mx.xcd_sh = MODE == LNSHIP_SUM32 ? xcd_shift((uint64_t)grid.x * grid.y * grid.z, cus) : 0;
    grid.x <<= mx.xcd_sh;
    hipLaunchKernelGGL((k_mm16<MODE, NC, PF, XL, CG, W>), grid, dim3(k_block * CG), lds, st, mx, T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

template <int MODE, int NC, int CG>
static int launch_mm16_x(const mm_args16 &m, const dev_tables &T, int64_t nslices, bool xl, int cus, hipStream_t st) {
    return xl ? launch_mm16<MODE, NC, true, CG>(m, T, nslices, cus, st) : launch_mm16<MODE, NC, false, CG>(m, T, nslices, cus, st);
}

template <int MODE>
static int dispatch_mm16(const mm_args16 &m, const dev_tables &T, int64_t nslices, const mm16_shape &sh,
                         int cus, hipStream_t st) {
    if constexpr (MODE == LNSHIP_SUM32) {
        // column groups: more waves per SIMD where the tables allow one
        // workgroup per CU
        switch (sh.nc * 10 + sh.cg) {
            case 12: return launch_mm16_x<MODE, 1, 2>(m, T, nslices, sh.xl, cus, st);
            case 14: return launch_mm16_x<MODE, 1, 4>(m, T, nslices, sh.xl, cus, st);
            case 24: return launch_mm16_x<MODE, 2, 4>(m, T, nslices, sh.xl, cus, st);
            case 44: return launch_mm16_x<MODE, 4, 4>(m, T, nslices, sh.xl, cus, st);
            case 84: return launch_mm16_x<MODE, 8, 4>(m, T, nslices, sh.xl, cus, st);
            default:
                if (sh.xl && narrow_mm(m.M * m.N * nslices, cus))
                    return launch_mm16<MODE, 1, true, 1, 16>(m, T, nslices, cus, st);
                return launch_mm16_x<MODE, 1, 1>(m, T, nslices, sh.xl, cus, st);
        }
    } else {
        switch (sh.nc) {
            case 8: return launch_mm16_x<MODE, 8, 1>(m, T, nslices, sh.xl, cus, st);
            case 4: return launch_mm16_x<MODE, 4, 1>(m, T, nslices, sh.xl, cus, st);
            default:
                if (sh.xl) switch (narrow_w(MODE, m.M * m.N * nslices, cus)) {
                        case 4:
                            if constexpr (MODE == LNSHIP_LPVIP) return launch_mm16<MODE, 1, true, 1, 4>(m, T, nslices, cus, st);
                            break;
                        case 8:
                            if constexpr (MODE == LNSHIP_LPVIP) return launch_mm16<MODE, 1, true, 1, 8>(m, T, nslices, cus, st);
                            break;
                        case 16: return launch_mm16<MODE, 1, true, 1, 16>(m, T, nslices, cus, st);
                        case 32: return launch_mm16<MODE, 1, true, 1, 32>(m, T, nslices, cus, st);
                        default: break;
                    }
                return launch_mm16_x<MODE, 1, 1>(m, T, nslices, sh.xl, cus, st);
        }
    }
}

// LDS of a k_mm32 launch: the single-chain image, and with XL the
// activation row's codes (and the prefetch past its last group)
static int64_t mm32_lds(bool xl, int64_t kp) { return k_lds_tab32 + (xl ? kp * 4 + 64 : 0); }
// whether an XL launch of rows of kp codes fits LDS
static bool mm32_xl_fits(int64_t kp) { return mm32_lds(true, kp) <= k_lds_bytes - k_lds_static; }

template <int NC, int CG, int W = 64, bool XL = false>
static int launch_mm32(const mm_args32 &m, const dev_tables &T, int64_t nslices, int cus, hipStream_t st) {
    // prefetch depth within 128 VGPRs at four waves per SIMD
    constexpr int PF = NC == 1 ? (CG >= 4 ? 2 : 4) : 1;
    const int lds = (int)mm32_lds(XL, m.kp);
    if (int rc = set_lds(k_mm32<NC, PF, CG, W, XL>, lds)) return rc;
    constexpr int rows = W < 64 ? k_block / 64 * W : k_block;   // rows per workgroup
    dim3 grid((unsigned)((m.M + rows - 1) / rows), (unsigned)((m.N + NC * CG - 1) / (NC * CG)), (unsigned)nslices);
    if (grid.x > 2147483647u || grid.y > 65535u) return fail(LNSHIP_ERANGE, "mul_mat: grid too large%s");
    mm_args32 mx = m;
    mx.xcd_sh = xcd_shift((uint64_t)grid.x * grid.y * grid.z, cus);
    grid.x <<= mx.xcd_sh;
    hipLaunchKernelGGL((k_mm32<NC, PF, CG, W, XL>), grid, dim3(k_block * CG), lds, st, mx, T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

template <int MODE>
static int launch_rms16(const float *src, const float *w, float *dst, int64_t ncols, int64_t nrows, float eps,
                        uint16_t seed, const uint16_t *state, uint64_t offset, const dev_tables &T, int cus,
                        hipStream_t st) {
    const int64_t rs = (ncols + 7) & ~(int64_t)7;
    const int rb = rows_per_block(row_tables_bytes<MODE>(), rs, 2, nrows, cus);
    if (rb < 1) return fail(LNSHIP_ERANGE, "rms_norm: row too long for LDS%s");
    const int lds = ((row_tables_bytes<MODE>() + 15) & ~15) + (int)(rb * rs * 2);
    if (int rc = set_lds(k_rms16<MODE>, lds)) return rc;
    hipLaunchKernelGGL(k_rms16<MODE>, dim3((unsigned)((nrows + rb - 1) / rb)), dim3(k_block), lds, st, src, w, dst,
                       ncols, nrows, rb, eps, (uint32_t)seed, state, offset, T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

static int check_sm(const lnship_soft_max_args *a) {
    if (!a) return fail(LNSHIP_EINVAL, "soft_max: null args%s");
    for (int i = 0; i < 4; i++)
        if (a->src_ne[i] < 0) return fail(LNSHIP_EINVAL, "soft_max: bad shape%s");
    if (a->mask) {
        for (int i = 0; i < 4; i++)
            if (a->mask_ne[i] <= 0) return fail(LNSHIP_EINVAL, "soft_max: bad mask shape%s");
        if (a->mask_ne[0] != a->src_ne[0] || a->mask_ne[1] < a->src_ne[1])
            return fail(LNSHIP_EINVAL, "soft_max: mask does not cover the rows%s");
    }
    return 0;
}

template <int MODE>
static int attn16_lds(int64_t hd, int64_t n_kv) {
    return mm_xl_offset<MODE>() + (int)(2 * ((hd + 7) & ~(int64_t)7) + 4 * ((n_kv + 7) & ~(int64_t)7));
}

template <int MODE>
static int launch_attn16(const attn_args &m, int64_t nh, const dev_tables &T, hipStream_t st) {
    const int lds = attn16_lds<MODE>(m.hd, m.n_kv);
    if (int rc = set_lds(k_attn16<MODE>, lds)) return rc;
    hipLaunchKernelGGL(k_attn16<MODE>, dim3(attn_grid(nh)), dim3(k_block), lds, st, m, T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

// LDS of a k_attn32 launch: the single-chain image, the query, the scores
// and the probabilities' codes (4 bytes each)
static int64_t attn32_lds(int64_t hd, int64_t n_kv) {
    return k_lds_tab32 + 4 * ((hd + 7) & ~(int64_t)7) + 8 * ((n_kv + 7) & ~(int64_t)7);
}

// cells of lnship16_attn_decode with head_dim up to 256
template <int MODE>
static int64_t max_attn_kv() {
    return ((k_lds_bytes - k_lds_static - attn16_lds<MODE>(256, 0)) / 4) & ~(int64_t)7;
}

// the dynamic LDS of a k_attn16 launch (64-bit: head_dim may be up to 4096)
static int64_t attn16_lds_mode(int mode, int64_t hd, int64_t n_kv) {
    const int64_t off = mode == LNSHIP_BASE ? mm_xl_offset<LNSHIP_BASE>()
                        : mode == LNSHIP_MONTE ? mm_xl_offset<LNSHIP_MONTE>()
                        : mode == LNSHIP_LPVIP ? mm_xl_offset<LNSHIP_LPVIP>()
                                               : mm_xl_offset<LNSHIP_SUM32>();
    return off + 2 * ((hd + 7) & ~(int64_t)7) + 4 * ((n_kv + 7) & ~(int64_t)7);
}

template <int MODE>
static int launch_sm16(sm_args &m, int64_t nrows, const dev_tables &T, int cus, hipStream_t st) {
    const int64_t rs = (m.n + 7) & ~(int64_t)7;
    m.rb = rows_per_block(row_tables_bytes<MODE>(), rs, 2, nrows, cus);
    if (m.rb < 1) return fail(LNSHIP_ERANGE, "soft_max: row too long for LDS%s");
    const int lds = ((row_tables_bytes<MODE>() + 15) & ~15) + (int)(m.rb * rs * 2);
    if (int rc = set_lds(k_softmax16<MODE>, lds)) return rc;
    hipLaunchKernelGGL(k_softmax16<MODE>, dim3((unsigned)((nrows + m.rb - 1) / m.rb)), dim3(k_block), lds, st, m, T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

// ---- dependent-latency probe ------------------------------------------------
// The floor under an LNS addition chain on one wave: RT dependent LDS reads
// per step (each read's value is the next read's byte address: a pointer
// chase through a permutation, no address arithmetic), then V dependent VALU
// operations (v_xor keeps the address in the table).  One workgroup of one
// wave, as a decode GEMV's chain lane runs.
template <int RT, int V>
__global__ __launch_bounds__(64) void k_chain_probe(int64_t steps, uint32_t *out) {
    __shared__ uint32_t t[4096];
    for (int i = threadIdx.x; i < 4096; i += 64) t[i] = ((uint32_t)(i * 97 + 13) & 4095u) << 2;
    __syncthreads();
    uint32_t x = (threadIdx.x * 61u & 4095u) << 2;
    const char *base = reinterpret_cast<const char *>(t);
    for (int64_t s = 0; s < steps; s += 8) {   // steps: a multiple of 8
#pragma unroll
        for (int u = 0; u < 8; u++) {
#pragma unroll
            for (int r = 0; r < RT; r++) x = *reinterpret_cast<const uint32_t *>(base + x);
#pragma unroll
            for (int v = 0; v < V; v++) asm volatile("v_xor_b32 %0, 4, %0" : "+v"(x));
        }
    }
    out[threadIdx.x] = x;
}

}  // namespace lnship

using namespace lnship;

// ===================================================================== C ABI ==

template <int W, int OP>
static int binary_common(const float *a, const float *b, int64_t n, int64_t nb, float *dst, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (n < 0 || nb <= 0) return fail(LNSHIP_EINVAL, OP == 0 ? "add: bad length%s" : "mul: bad length%s");
    if (n == 0) return 0;
    hipLaunchKernelGGL((k_binary<W, OP>), dim3(grid_for(n)), dim3(k_block), 0, (hipStream_t)stream, a, b, n, nb,
                       dst, s->T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

template <int W>
static int scale_common(const float *src, float *dst, int64_t n, float sc, float b, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (n < 0) return fail(LNSHIP_EINVAL, "scale: bad length%s");
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_scale<W>, dim3(grid_for(n)), dim3(k_block), 0, (hipStream_t)stream, src, dst, n, sc, b,
                       s->T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

template <int W>
static int swiglu_common(const float *gate, int64_t gate_ld, const float *up, int64_t up_ld, float *dst,
                         int64_t ncols, int64_t nrows, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (ncols < 0 || nrows < 0 || gate_ld < ncols || up_ld < ncols) return fail(LNSHIP_EINVAL, "swiglu: bad shape%s");
    if (ncols == 0 || nrows == 0) return 0;
    hipLaunchKernelGGL(k_swiglu<W>, dim3(grid_for(ncols * nrows)), dim3(k_block), 0, (hipStream_t)stream, gate,
                       gate_ld, up, up_ld, dst, ncols, nrows, s->T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

template <int W>
static int rope_common(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                       int n_dims, int neox, const float *cos_sin, float *dst, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (n_dims <= 0 || n_dims % 2 || n_dims > ne0 || x_ld < nhead * ne0 || ntok < 0 || nhead < 0)
        return fail(LNSHIP_EINVAL, "rope: bad shape%s");
    const int64_t n = ntok * nhead * (n_dims / 2 + ne0 - n_dims);
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_rope<W>, dim3(grid_for(n)), dim3(k_block), 0, (hipStream_t)stream, x, x_ld, pos, ntok,
                       nhead, ne0, n_dims, neox, cos_sin, dst, s->T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

template <int W>
static int store_kv_common(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                           int rope_n_dims, const float *cos_sin, typename fmt_t<W>::code_t *cache, int64_t cache_m,
                           int64_t cache_slice, int cache_transposed, const int32_t *seq, int64_t seq_stride,
                           void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (rope_n_dims < 0 || rope_n_dims % 2 || rope_n_dims > ne0 || x_ld < nhead * ne0 || ntok < 0 || nhead < 0)
        return fail(LNSHIP_EINVAL, "store_kv: bad shape%s");
    if (!cache_transposed && ne0 % 8) return fail(LNSHIP_EINVAL, "store_kv: head size not a multiple of 8%s");
    if (seq && seq_stride < 0) return fail(LNSHIP_EINVAL, "store_kv: negative sequence stride%s");
    const int64_t n = ntok * nhead * ne0;
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_store_kv<W>, dim3(grid_for(n)), dim3(k_block), 0, (hipStream_t)stream, x, x_ld, pos, ntok,
                       nhead, ne0, rope_n_dims, cos_sin, cache, cache_m, cache_slice, cache_transposed, seq, seq_stride,
                       s->T, s->index_err);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

template <int W>
static int rope_store_kv_common(const lnship_qkv_store_args *a, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (!a || a->ntok < 0 || a->n_head < 0 || a->n_head_kv < 0 || a->head_dim <= 0 || a->head_dim % 8 ||
        a->rope_n_dims <= 0 || a->rope_n_dims % 2 || a->rope_n_dims > a->head_dim ||
        a->qkv_ld < (a->n_head + 2 * a->n_head_kv) * a->head_dim || (a->seq && a->seq_stride < 0))
        return fail(LNSHIP_EINVAL, "rope_store_kv: bad shape%s");
    const int64_t hd = a->head_dim, nd = a->rope_n_dims;
    const int64_t n = a->ntok * (a->n_head * (nd / 2 + hd - nd) + 2 * a->n_head_kv * hd);
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_rope_store_kv<W>, dim3(grid_for(n)), dim3(k_block), 0, (hipStream_t)stream, *a, s->T,
                       s->index_err);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

extern "C" {

const char *lnship_last_error(void) { return t_err.c_str(); }

const char *lnship_version(void) { return "lnship 0.1: xlns16 (table, alt) + xlns32 (alt) for gfx950"; }

static bool pos32_image(const int32_t *tab, std::vector<int32_t> &img);
static std::vector<int32_t> g_pos32_host;   // the positive-sum adder's pair image, for tests

const void *lnship_host_table(const char *name, size_t *bytes) {
    {
        std::lock_guard<std::mutex> lock(g_mutex);
        if (!g_host) {
            g_host = new host_tables;
            build_host_tables(*g_host);
        }
        if (g_pos32_host.empty() && std::strcmp(name, "pos32") == 0 && !pos32_image(g_host->tab32, g_pos32_host)) {
            g_pos32_host.clear();
            fail(LNSHIP_EINVAL, "sb slopes outside the positive-sum adder's 24-bit range%s");
            return nullptr;
        }
    }
    if (std::strcmp(name, "pos32") == 0) {
        if (bytes) *bytes = g_pos32_host.size() * sizeof(int32_t);
        return g_pos32_host.data();
    }
    struct { const char *n; const void *p; size_t b; } t[] = {
        {"cvt16", g_host->cvt16, sizeof g_host->cvt16},
        {"rev16", g_host->rev16, sizeof g_host->rev16},
        {"gauss16", g_host->gauss16, sizeof g_host->gauss16},
        {"gauss16m", g_host->gauss16m, sizeof g_host->gauss16m},
        {"exp16", g_host->exp16, sizeof g_host->exp16},
        {"sig16", g_host->sig16, sizeof g_host->sig16},
        {"tab32", g_host->tab32, sizeof g_host->tab32},
        {"lfsr_seq", g_host->lfsr_seq, sizeof g_host->lfsr_seq},
    };
    for (auto &e : t)
        if (std::strcmp(e.n, name) == 0) {
            if (bytes) *bytes = e.b;
            return e.p;
        }
    fail(LNSHIP_EINVAL, "unknown table %s", name);
    return nullptr;
}

// The LDS image of the xlns32 adder tables after the descriptors (which hold
// LDS addresses, so each workgroup forms them).  -dlo[dl] (>= 0), with 36
// binades in place of the db-at-zero entry; dhi as pairs (th2, nth), th2 =
// (dh << 12) + dhi[dh], the first half of the cotransformation's e, and nth =
// -dhi[dh] (>= 0), less the part the result adds.  dh = 0 gets (13 binades,
// 2^31 - 1).  e = th2 - dlo[dl] then lies in the essential zero's sbf
// zeros (24 to 38 binades) on the dh = 0 lanes (-dlo[dl] in [11.5, 23.6]
// binades for dl > 0) and on the dl = 0 lanes (th2 >= -11.6 binades for
// dh > 0), and only at d = 0 reaches 13 + 36 = 49 binades, the node that
// clamps the log to 0.  The addend min(nth, -dlo[dl], cap) is -dlo[dl] where
// dh = 0, else -dhi[dh] (db rises with the distance and dh << 12 > dl, so
// -dhi[dh] < -dlo[dl]).  Then the interpolation tables sb, sbf (extended),
// db, dbf, and a zero pair.
// Returns false when the tables break a bound the layout relies on.  dec:
// the single-chain step's image, whose dhi pairs hold ksb - th2 in place of th2.
static bool lds32_image(const int32_t *tab, std::vector<int32_t> &img, bool dec) {
    // (word kl_dlo of the LDS copy is word 0 of the image)
    img.assign(kl_end - kl_dlo, 0);
    int32_t *w = img.data() - kl_dlo;
    for (int i = 1; i < k32_co_n; i++) w[kl_dlo + i] = -tab[k32_off_dlo + i];
    w[kl_dlo] = (int32_t)k32_co_l0;
    for (int i = 0; i < k32_co_n; i++) {
        const int32_t h = tab[k32_off_dhi + i];
        const int32_t th2 = i == 0 ? (int32_t)k32_co_h0 : h + (i << k32_co_sh);
        w[kl_dhi + 2 * i] = dec ? (int32_t)(k32_sb_end - 1u) - th2 : th2;
        // dh = 0: above every -dlo[dl], so the minimum takes -dlo[dl] there,
        // and -dhi[dh] elsewhere (db rises with the distance, dh << 12 > dl)
        w[kl_dhi + 2 * i + 1] = i == 0 ? 0x7fffffff : -h;
    }
    for (int i = 0; i < k32_sb_n; i++) w[kl_sb + i] = tab[k32_off_sb + i];
    for (int i = 0; i < k32_sb_fn; i++) w[kl_sbf + i] = tab[k32_off_sbf + i];
    // past the essential zero sbf reads 0 up to the exact-cancellation node,
    // whose pair drives any sum below 0 (the log clamps to 0)
    const int cancel = (int)((k32_co_cancel - k32_sb_end) >> k32_sb_fsh);
    w[kl_sbf + cancel] = w[kl_sbf + cancel + 1] = -0x7fffffff;
    for (int i = 0; i < k32_db_n; i++) w[kl_db + i] = tab[k32_off_db + i];
    for (int i = 0; i < k32_db_fn; i++) w[kl_dbf + i] = tab[k32_off_dbf + i];
    // the bounds: every e short of the segment before the cancellation node
    // and past the essential zero on the sentinel lanes; -dhi below -dlo
    int64_t nlo_min = INT64_MAX, nlo_max = INT64_MIN, th2_min = INT64_MAX, th2_max = INT64_MIN, nth_max = INT64_MIN;
    for (int i = 1; i < k32_co_n; i++) {
        const int64_t th2 = dec ? (int64_t)(k32_sb_end - 1u) - w[kl_dhi + 2 * i] : w[kl_dhi + 2 * i];
        nlo_min = std::min<int64_t>(nlo_min, w[kl_dlo + i]);
        nlo_max = std::max<int64_t>(nlo_max, w[kl_dlo + i]);
        th2_min = std::min<int64_t>(th2_min, th2);
        th2_max = std::max<int64_t>(th2_max, th2);
        nth_max = std::max<int64_t>(nth_max, w[kl_dhi + 2 * i + 1]);
    }
    const int64_t seg = (int64_t)k32_co_cancel - (1 << k32_sb_fsh), ess = k32_esszer;
    return w[kl_sbf + k32_sb_fn - 1] == 0 && (int64_t)k32_co_h0 + nlo_min >= ess &&
           (int64_t)k32_co_h0 + nlo_max < seg && th2_min + (int64_t)k32_co_l0 >= ess &&
           th2_max + (int64_t)k32_co_l0 < seg && th2_max + nlo_max < seg && th2_min + nlo_min >= 0 &&
           nth_max < nlo_min && nth_max < (int64_t)k32_co_l0;
}

// The positive-sum adder's pair image (k_lds_pos32): for each sb grid
// interval its first node and its slope scaled for v_mul_hi_i32_i24.
// Returns false when a scaled slope leaves the 24-bit signed range or the
// far grid does not end in zeros at the essential zero.
static bool pos32_image(const int32_t *tab, std::vector<int32_t> &img) {
    img.assign(2 * kp32_pairs, 0);
    bool ok = true;
    auto put = [&](int p, int32_t t0, int32_t t1, int sc) {
        const int64_t a = (int64_t)(t1 - t0) * ((int64_t)1 << sc);
        ok = ok && a >= -(1 << 23) && a < (1 << 23);
        img[2 * p] = t0;
        img[2 * p + 1] = (int32_t)a;
    };
    for (int i = 0; i < kp32_near; i++) put(i, tab[k32_off_sb + i], tab[k32_off_sb + i + 1], kp32_near_slope);
    for (int j = 0; j < kp32_far; j++)
        put(kp32_near + j, j < k32_sb_fn ? tab[k32_off_sbf + j] : 0, j + 1 < k32_sb_fn ? tab[k32_off_sbf + j + 1] : 0,
            kp32_far_slope);
    return ok && tab[k32_off_sbf + k32_sb_fn - 1] == 0;
}

int lnship_init(void) {
    int dev = 0;
    if (int rc = current_device(&dev)) return rc;
    if (!lnship_host_table("cvt16", nullptr)) return LNSHIP_EINVAL;
    std::lock_guard<std::mutex> lock(g_mutex);
    device_state &s = g_devices[dev];
    if (s.ready) return 0;
    dev_tables T{};
    if (int rc = upload(g_host->cvt16, 1u << 17, &T.cvt16)) return rc;
    if (int rc = upload(g_host->rev16, 1u << 16, &T.rev16)) return rc;
    {
        // an xlns16 code through F32 and back (the round trip between graph
        // nodes), as x16_from_f32(cvt16, rev16[c]) forms it on the device
        std::vector<uint16_t> rho(1u << 16);
        for (uint32_t c = 0; c < (1u << 16); c++) {
            uint32_t bits;
            std::memcpy(&bits, &g_host->rev16[c], 4);
            rho[c] = g_host->cvt16[bits >> 15];
        }
        if (int rc = upload(rho.data(), rho.size(), &T.rho16)) return rc;
    }
    if (int rc = upload(g_host->gauss16, 2 * k16_gauss_n, &T.gauss16)) return rc;
    {
        // the Monte adder's LDS image: host_tables::gauss16m with db's dither
        // entries (64 - F, -1) as (-F, 63): the adder then draws 63 - r for
        // db, so that every entry's second word is a plain mask (0 or 63)
        std::vector<int32_t> mimg(g_host->gauss16m, g_host->gauss16m + 4 * k16_mc_n);
        for (int d = 0; d < k16_mc_n; d++)
            if (mimg[4 * d + 3] == -1) {
                mimg[4 * d + 2] -= 64;
                mimg[4 * d + 3] = 63;
            }
        if (int rc = upload(mimg.data(), mimg.size(), &T.gauss16m)) return rc;
    }
    if (int rc = upload(g_host->exp16, 1u << 16, &T.exp16)) return rc;
    if (int rc = upload(g_host->lpdb, 3 * k_lp_n, &T.lpdb)) return rc;
    if (int rc = upload(g_host->sig16, 1u << 16, &T.sig16)) return rc;
    if (int rc = upload(g_host->tab32, (size_t)k32_tab_n, &T.tab32)) return rc;
    {
        std::vector<int32_t> img;
        if (!lds32_image(g_host->tab32, img, false))
            return fail(LNSHIP_EINVAL, "init: xlns32 tables outside the bounds of their LDS layout%s");
        if (int rc = upload(img.data(), img.size(), &T.lds32)) return rc;
        if (!lds32_image(g_host->tab32, img, true))
            return fail(LNSHIP_EINVAL, "init: xlns32 tables outside the bounds of their LDS layout%s");
        if (int rc = upload(img.data(), img.size(), &T.lds32d)) return rc;
        if (!pos32_image(g_host->tab32, img))
            return fail(LNSHIP_EINVAL, "init: sb slopes outside the positive-sum adder's 24-bit range%s");
        if (int rc = upload(img.data(), img.size(), &T.pos32)) return rc;
    }
    if (int rc = upload(g_host->lfsr_seq, 65536, &T.lfsr_seq)) return rc;
    if (int rc = upload(g_host->lfsr_log, 65536, &T.lfsr_log)) return rc;
    s.T = T;
    LNSHIP_HIP(hipDeviceGetAttribute(&s.cus, hipDeviceAttributeMultiprocessorCount, dev));
    LNSHIP_HIP(hipMalloc((void **)&s.index_err, 2 * sizeof(unsigned long long)));
    LNSHIP_HIP(hipMemset(s.index_err, 0, 2 * sizeof(unsigned long long)));
    // this device's copy of the fixed scratch (the device is current here)
    void *fixed = nullptr;
    LNSHIP_HIP(hipGetSymbolAddress(&fixed, HIP_SYMBOL(scratch)));
    if (!fixed) return fail(LNSHIP_EDEVICE, "no address for the fixed scratch%s");
    s.fixed_scratch = fixed;
    s.ready = true;
    return 0;
}

int lnship_chain_probe(int round_trips, int valu_ops, int64_t steps, void *stream, double *ns_per_step) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (!ns_per_step || steps <= 0 || steps > ((int64_t)1 << 32)) return fail(LNSHIP_EINVAL, "chain_probe: bad steps%s");
    steps = (steps + 7) & ~(int64_t)7;
    auto launch = [&](hipStream_t st) -> int {
        void *xs = nullptr;
        if (int rc = grow_scratch(s, 256, &xs, st)) return rc;
        uint32_t *o = static_cast<uint32_t *>(xs);
        switch (round_trips * 10 + valu_ops) {
            case 10: hipLaunchKernelGGL((k_chain_probe<1, 0>), dim3(1), dim3(64), 0, st, steps, o); break;
            case 20: hipLaunchKernelGGL((k_chain_probe<2, 0>), dim3(1), dim3(64), 0, st, steps, o); break;
            case 21: hipLaunchKernelGGL((k_chain_probe<2, 1>), dim3(1), dim3(64), 0, st, steps, o); break;
            case 1: hipLaunchKernelGGL((k_chain_probe<0, 1>), dim3(1), dim3(64), 0, st, steps, o); break;
            case 8: hipLaunchKernelGGL((k_chain_probe<0, 8>), dim3(1), dim3(64), 0, st, steps, o); break;
            default: return fail(LNSHIP_EINVAL, "chain_probe: (round_trips, valu_ops) not one of (1,0) (2,0) (2,1) (0,1) (0,8)%s");
        }
        LNSHIP_HIP(hipGetLastError());
        return 0;
    };
    hipStream_t st = (hipStream_t)stream;
    if (int rc = launch(st)) return rc;   // warm-up
    hipEvent_t e0, e1;
    LNSHIP_HIP(hipEventCreate(&e0));
    LNSHIP_HIP(hipEventCreate(&e1));
    LNSHIP_HIP(hipEventRecord(e0, st));
    int rc = launch(st);
    LNSHIP_HIP(hipEventRecord(e1, st));
    LNSHIP_HIP(hipEventSynchronize(e1));
    float ms = 0.0f;
    LNSHIP_HIP(hipEventElapsedTime(&ms, e0, e1));
    LNSHIP_HIP(hipEventDestroy(e0));
    LNSHIP_HIP(hipEventDestroy(e1));
    if (rc) return rc;
    *ns_per_step = (double)ms * 1e6 / (double)steps;
    return 0;
}

uint16_t lnship_lfsr_jump(uint16_t st, uint64_t n) {
    for (uint64_t i = n % 65535u; i > 0; i--) st = (uint16_t)((st >> 1) ^ ((st & 1u) ? 0xB400u : 0u));
    return st;
}

} // extern "C"

namespace lnship {
__global__ void k_lfsr_advance(uint16_t *state, uint64_t draws, dev_tables T) {
    if (threadIdx.x == 0) *state = (uint16_t)lfsr_jump(T, *state, draws);
}
} // namespace lnship

extern "C" {

int lnship_lfsr_advance(uint16_t *lfsr, uint64_t draws, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (!lfsr) return fail(LNSHIP_EINVAL, "lfsr_advance: null state%s");
    hipLaunchKernelGGL(k_lfsr_advance, dim3(1), dim3(64), 0, (hipStream_t)stream, lfsr, draws, s->T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

uint64_t lnship16_mul_mat_draws(int mode, int64_t K, int64_t M, int64_t N, int64_t ne12, int64_t ne13) {
    if (mode != LNSHIP_MONTE || K <= 0) return 0;
    return (uint64_t)ne12 * (uint64_t)ne13 * (uint64_t)M * (uint64_t)N * (uint64_t)(K - 1);
}
uint64_t lnship16_soft_max_draws(int mode, int64_t ncols, int64_t nrows) {
    return mode == LNSHIP_MONTE && ncols > 0 ? (uint64_t)nrows * (uint64_t)(ncols - 1) : 0;
}
uint64_t lnship16_rms_norm_draws(int mode, int64_t ncols, int64_t nrows) {
    return mode == LNSHIP_MONTE ? (uint64_t)nrows * (uint64_t)ncols : 0;
}

int lnship16_from_f32(const float *src, uint16_t *dst, int64_t n, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (n < 0) return fail(LNSHIP_EINVAL, "negative length%s");
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_from_f32_16, dim3(grid_for(n, 4)), dim3(k_block), 0, (hipStream_t)stream, src, dst, n,
                       s->T.cvt16);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship16_to_f32(const uint16_t *src, float *dst, int64_t n, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (n < 0) return fail(LNSHIP_EINVAL, "negative length%s");
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_to_f32_16, dim3(grid_for(n, 4)), dim3(k_block), 0, (hipStream_t)stream, src, dst, n,
                       s->T.rev16);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship32_from_f32(const float *src, uint32_t *dst, int64_t n, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (n < 0) return fail(LNSHIP_EINVAL, "negative length%s");
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_from_f32_32, dim3(grid_for(n, 4)), dim3(k_block), 0, (hipStream_t)stream, src, dst, n);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship32_to_f32(const uint32_t *src, float *dst, int64_t n, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (n < 0) return fail(LNSHIP_EINVAL, "negative length%s");
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_to_f32_32, dim3(grid_for(n, 4)), dim3(k_block), 0, (hipStream_t)stream, src, dst, n);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}


// Packs nslices weight slices, each M rows of K (row stride src_ld, slice
// stride src_slice), into the k8-interleaved cache layout (Kp * M codes per
// slice, Kp = K rounded up to 8).
int lnship16_pack(const void *src, int src_is_f16, int64_t src_ld, int64_t src_slice, uint16_t *dst, int64_t K,
                  int64_t M, int64_t nslices, void *stream) {
    return pack_common(0, src, src_is_f16, src_ld, src_slice, dst, K, M, nslices, stream);
}
int lnship32_pack(const void *src, int src_is_f16, int64_t src_ld, int64_t src_slice, uint32_t *dst, int64_t K,
                  int64_t M, int64_t nslices, void *stream) {
    return pack_common(1, src, src_is_f16, src_ld, src_slice, dst, K, M, nslices, stream);
}

// the xlns16 code of v, as the device's conversion table gives it
static uint32_t host_cvt16(float v) {
    const uint16_t *cvt = static_cast<const uint16_t *>(lnship_host_table("cvt16", nullptr));
    uint32_t b;
    std::memcpy(&b, &v, 4);
    return cvt[b >> 15];
}

int lnship16_mul_mat(int mode, const lnship_mul_mat_args *a, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (mode < 0 || mode > 3) return fail(LNSHIP_EINVAL, "unknown summation mode%s");
    if (int rc = check_mm(a)) return rc;
    if (a->M == 0 || a->N == 0) return 0;
    if (a->K > (int64_t)1 << 30) return fail(LNSHIP_ERANGE, "mul_mat: K beyond 2^30%s");
    const int64_t nslices = a->ne12 * a->ne13;
    const int64_t kp = (a->K + 7) & ~(int64_t)7;
    const int64_t xld = a->x_ld ? a->x_ld : a->K;
    const int64_t xslice = a->x_slice ? a->x_slice : a->N * xld;
    hipStream_t st = (hipStream_t)stream;
    // activations converted inside the GEMV when NC rows fit in LDS next to
    // the tables, else by k_act into scratch first
    const mm16_shape sh = mm16_choose(mode, a->M, a->N, nslices, kp, s->cus);
    if (a->rms_norm_w || a->glu_up) {
        // the nodes before the product run in the activation staging
        if (a->rms_norm_w && a->glu_up) return fail(LNSHIP_EINVAL, "mul_mat: rms_norm_w and glu_up together%s");
        if (nslices != 1 || a->K < 1)
            return fail(LNSHIP_EINVAL, "mul_mat: rms_norm_w / glu_up need one activation slice and K >= 1%s");
        if (!sh.xl) return fail(LNSHIP_ERANGE, "mul_mat: rows too long to stage beside the tables for "
                                               "rms_norm_w / glu_up%s");
    }
    void *xs = nullptr;
    if (!sh.xl) {
        if (int rc = grow_scratch(s, (size_t)std::max<int64_t>(1, nslices * a->N * kp) * 2, &xs, st)) return rc;
        if (kp > 0) {
            dim3 g(grid_for(a->N * kp, 2), (unsigned)nslices);
            hipLaunchKernelGGL(k_act<0>, g, dim3(k_block), 0, st, a->x, xld, xslice, xs, a->N, a->K, kp, s->T.cvt16);
            LNSHIP_HIP(hipGetLastError());
        }
    }
    const int64_t wms = a->w_mstride ? a->w_mstride : a->M;
    const int64_t dld = a->dst_ld ? a->dst_ld : a->M;
    mm_args16 m{(const uint16_t *)a->w, (const uint16_t *)xs, a->x, a->dst, a->K, kp, a->M, a->N, xld, xslice,
                a->ne02, a->ne12, a->ne12 / a->ne02, a->ne13 / a->ne03,
                wms, a->w_slice ? a->w_slice : kp * wms, dld, a->dst_slice ? a->dst_slice : a->N * dld,
                a->monte_seed, a->monte_state, a->monte_offset};
    m.resid = a->residual;
    m.glu_up = a->glu_up;
    if (a->rms_norm_w) {
        m.norm = a->rms_norm_w;
        m.rms_ik = host_cvt16(1.0f / (float)a->K);
        m.rms_eps = host_cvt16(a->rms_eps);
        m.rms_seed = a->rms_seed;
        m.rms_offset = a->rms_offset;
    }
    switch (mode) {
        case LNSHIP_BASE: return dispatch_mm16<LNSHIP_BASE>(m, s->T, nslices, sh, s->cus, st);
        case LNSHIP_MONTE: return dispatch_mm16<LNSHIP_MONTE>(m, s->T, nslices, sh, s->cus, st);
        case LNSHIP_LPVIP: return dispatch_mm16<LNSHIP_LPVIP>(m, s->T, nslices, sh, s->cus, st);
        default: return dispatch_mm16<LNSHIP_SUM32>(m, s->T, nslices, sh, s->cus, st);
    }
}


int lnship16_swiglu_mul_mat(int mode, const float *gate, const float *up, const void *w, const float *residual,
                            float *dst, int64_t K, int64_t M, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (mode == LNSHIP_MONTE)
        return fail(LNSHIP_EINVAL, "swiglu_mul_mat: Monte draws run in graph order; run the two nodes%s");
    if (mode < 0 || mode > 3) return fail(LNSHIP_EINVAL, "unknown summation mode%s");
    if (!gate || !up || !w || !dst || K < 1 || M < 0) return fail(LNSHIP_EINVAL, "swiglu_mul_mat: bad argument%s");
    if (M == 0) return 0;
    const int64_t kp = (K + 7) & ~(int64_t)7;
    const mm16_shape sh = mm16_choose(mode, M, 1, 1, kp, s->cus);
    if (!sh.xl) return fail(LNSHIP_ERANGE, "swiglu_mul_mat: row too long for LDS%s");
    mm_args16 m{(const uint16_t *)w, nullptr, gate, dst, K, kp, M, 1, K, K, 1, 1, 1, 1, M, kp * M, M, M, 0, nullptr, 0};
    m.glu_up = up;
    m.resid = residual;
    hipStream_t st = (hipStream_t)stream;
    switch (mode) {
        case LNSHIP_BASE: return dispatch_mm16<LNSHIP_BASE>(m, s->T, 1, sh, s->cus, st);
        case LNSHIP_LPVIP: return dispatch_mm16<LNSHIP_LPVIP>(m, s->T, 1, sh, s->cus, st);
        default: return dispatch_mm16<LNSHIP_SUM32>(m, s->T, 1, sh, s->cus, st);
    }
}

// The xlns32 product once its activation rows have a staging block xs of
// at least nslices * N * kp codes: k_act converts them (padding included, so
// xs needs no clearing), then the GEMV.
static int mul_mat32_staged(device_state *s, const lnship_mul_mat_args *a, void *xs, hipStream_t st) {
    const int64_t nslices = a->ne12 * a->ne13;
    const int64_t kp = (a->K + 7) & ~(int64_t)7;
    if (kp > 0) {
        dim3 g(grid_for(a->N * kp, 2), (unsigned)nslices);
        hipLaunchKernelGGL(k_act<1>, g, dim3(k_block), 0, st, a->x, a->x_ld ? a->x_ld : a->K,
                           a->x_slice ? a->x_slice : a->N * (a->x_ld ? a->x_ld : a->K), xs, a->N, a->K, kp,
                           s->T.cvt16);
        LNSHIP_HIP(hipGetLastError());
    }
    const int64_t wms = a->w_mstride ? a->w_mstride : a->M;
    const int64_t dld = a->dst_ld ? a->dst_ld : a->M;
    mm_args32 m{(const uint32_t *)a->w, (const uint32_t *)xs, a->dst, a->K, kp, a->M, a->N,
                a->ne02, a->ne12, a->ne12 / a->ne02, a->ne13 / a->ne03,
                wms, a->w_slice ? a->w_slice : kp * wms, dld, a->dst_slice ? a->dst_slice : a->N * dld};
    m.resid = a->residual;
    const mm16_shape sh = mm_shape_x32(m.M, m.N, nslices, kp, s->cus, 4);
    switch (sh.nc * 10 + sh.cg) {
        case 12: return launch_mm32<1, 2>(m, s->T, nslices, s->cus, st);
        case 14: return launch_mm32<1, 4>(m, s->T, nslices, s->cus, st);
        case 24: return launch_mm32<2, 4>(m, s->T, nslices, s->cus, st);
        case 44: return launch_mm32<4, 4>(m, s->T, nslices, s->cus, st);
        default:
            // one column: 16-row waves while they fill at most one wave slot
            // per SIMD (as the sum32 GEMV)
            if (narrow_mm(m.M * m.N * nslices, s->cus)) return launch_mm32<1, 1, 16>(m, s->T, nslices, s->cus, st);
            return launch_mm32<1, 1>(m, s->T, nslices, s->cus, st);
    }
}

// the nodes before the product that only lnship32_mul_mat takes in its launch
static int check_mm32_plain(const lnship_mul_mat_args *a) {
    if (a->rms_norm_w || a->glu_up)
        return fail(LNSHIP_EINVAL, "mul_mat_noalloc (LNS32): no rms_norm_w / glu_up%s");
    return 0;
}

int lnship32_mul_mat(const lnship_mul_mat_args *a, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (int rc = check_mm(a)) return rc;
    const int64_t nslices = a->ne12 * a->ne13;
    const int64_t kp = (a->K + 7) & ~(int64_t)7;
    if (a->rms_norm_w || a->glu_up) {
        if (a->rms_norm_w && a->glu_up) return fail(LNSHIP_EINVAL, "mul_mat: rms_norm_w and glu_up together%s");
        if (nslices != 1 || a->K < 1)
            return fail(LNSHIP_EINVAL, "mul_mat: rms_norm_w / glu_up need one activation slice and K >= 1%s");
    }
    if (a->M == 0 || a->N == 0) return 0;
    hipStream_t st = (hipStream_t)stream;
    // one column per workgroup (every decode shape) with the row beside the
    // tables: the launch converts its activations itself (and forms the
    // nodes before the product), no k_act launch
    const mm16_shape sh = mm_shape_x32(a->M, a->N, nslices, kp, s->cus, 4);
    const bool xl = sh.nc * 10 + sh.cg == 11 && kp > 0 && mm32_xl_fits(kp);
    if ((a->rms_norm_w || a->glu_up) && !xl)
        return fail(LNSHIP_ERANGE, "mul_mat: rows too long to stage beside the tables for rms_norm_w / glu_up%s");
    if (xl) {
        const int64_t wms = a->w_mstride ? a->w_mstride : a->M;
        const int64_t dld = a->dst_ld ? a->dst_ld : a->M;
        const int64_t xld = a->x_ld ? a->x_ld : a->K;
        mm_args32 m{(const uint32_t *)a->w, nullptr, a->dst, a->K, kp, a->M, a->N,
                    a->ne02, a->ne12, a->ne12 / a->ne02, a->ne13 / a->ne03,
                    wms, a->w_slice ? a->w_slice : kp * wms, dld, a->dst_slice ? a->dst_slice : a->N * dld};
        m.resid = a->residual;
        m.xf = a->x;
        m.x_ld = xld;
        m.x_slice = a->x_slice ? a->x_slice : a->N * xld;
        m.norm = a->rms_norm_w;
        m.eps = a->rms_eps;
        m.glu_up = a->glu_up;
        if (narrow_mm(m.M * m.N * nslices, s->cus)) return launch_mm32<1, 1, 16, true>(m, s->T, nslices, s->cus, st);
        return launch_mm32<1, 1, 64, true>(m, s->T, nslices, s->cus, st);
    }
    void *xs = nullptr;
    if (int rc = grow_scratch(s, (size_t)std::max<int64_t>(1, a->ne12 * a->ne13 * a->N * kp) * 4, &xs, st)) return rc;
    return mul_mat32_staged(s, a, xs, st);
}

int lnship32_mul_mat_noalloc(const lnship_mul_mat_args *a, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (int rc = check_mm(a)) return rc;
    if (int rc = check_mm32_plain(a)) return rc;
    if (a->M == 0 || a->N == 0) return 0;
    const int64_t kp = (a->K + 7) & ~(int64_t)7;
    const uint64_t need = (uint64_t)(a->ne12 * a->ne13) * (uint64_t)a->N * (uint64_t)kp * 4u;
    if (need > k_fixed_scratch_bytes)
        return fail(LNSHIP_ERANGE, "mul_mat_noalloc: ne12*ne13*N*round8(K) activation codes exceed the 1 Mi "
                                   "(4 MiB) fixed scratch%s");
    return mul_mat32_staged(s, a, s->fixed_scratch, (hipStream_t)stream);
}


static int check_mm_id(const lnship_mul_mat_id_args *a) {
    if (!a || a->K < 0 || a->M < 0 || a->n_expert <= 0 || a->n_expert_used < 0 || a->n_tokens < 0 || a->ne11 <= 0)
        return fail(LNSHIP_EINVAL, "mul_mat_id: bad shape%s");
    if (a->n_expert_used % a->ne11) return fail(LNSHIP_EINVAL, "mul_mat_id: slots do not broadcast over rows%s");
    if ((a->x_ld ? a->x_ld : a->K) < a->K) return fail(LNSHIP_EINVAL, "mul_mat_id: x_ld < K%s");
    if (a->ids_ld && a->ids_ld < a->n_expert_used) return fail(LNSHIP_EINVAL, "mul_mat_id: ids_ld < n_expert_used%s");
    if (a->n_expert_used * a->n_tokens > 65535) return fail(LNSHIP_ERANGE, "mul_mat_id: more than 65535 slots%s");
    if (a->K > (int64_t)1 << 30) return fail(LNSHIP_ERANGE, "mul_mat_id: K beyond 2^30%s");
    return 0;
}

// MUL_MAT_ID as a GEMV per (slot, token): grid slice z = t n_expert_used + s
// with one column, so the Monte draws follow the reference's (t, s, row) order
int lnship16_mul_mat_id(int mode, const lnship_mul_mat_id_args *a, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (mode < 0 || mode > 3) return fail(LNSHIP_EINVAL, "unknown summation mode%s");
    if (int rc = check_mm_id(a)) return rc;
    const int64_t nslices = a->n_expert_used * a->n_tokens;
    if (a->M == 0 || nslices == 0) return 0;
    const int64_t kp = (a->K + 7) & ~(int64_t)7, xld = a->x_ld ? a->x_ld : a->K;
    hipStream_t st = (hipStream_t)stream;
    const mm16_shape sh = mm16_choose(mode, a->M, 1, nslices, kp, s->cus);
    void *xs = nullptr;
    if (!sh.xl) {   // the distinct activation rows, converted once
        const int64_t rows = a->ne11 * a->n_tokens;
        if (int rc = grow_scratch(s, (size_t)std::max<int64_t>(1, rows * kp) * 2, &xs, st)) return rc;
        if (kp > 0) {
            hipLaunchKernelGGL(k_act<0>, dim3(grid_for(kp, 2), (unsigned)rows), dim3(k_block), 0, st, a->x, xld, xld,
                               xs, (int64_t)1, a->K, kp, s->T.cvt16);
            LNSHIP_HIP(hipGetLastError());
        }
    }
    mm_args16 m{(const uint16_t *)a->w, (const uint16_t *)xs, a->x, a->dst, a->K, kp, a->M, 1, xld, xld,
                1, a->n_expert_used, 1, 1, a->M, kp * a->M, a->M, a->M,
                a->monte_seed, a->monte_state, a->monte_offset,
                a->ids, a->ids_ld ? a->ids_ld : a->n_expert_used, a->ne11, a->n_expert, s->index_err};
    switch (mode) {
        case LNSHIP_BASE: return dispatch_mm16<LNSHIP_BASE>(m, s->T, nslices, sh, s->cus, st);
        case LNSHIP_MONTE: return dispatch_mm16<LNSHIP_MONTE>(m, s->T, nslices, sh, s->cus, st);
        case LNSHIP_LPVIP: return dispatch_mm16<LNSHIP_LPVIP>(m, s->T, nslices, sh, s->cus, st);
        default: return dispatch_mm16<LNSHIP_SUM32>(m, s->T, nslices, sh, s->cus, st);
    }
}

int lnship32_mul_mat_id(const lnship_mul_mat_id_args *a, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (int rc = check_mm_id(a)) return rc;
    const int64_t nslices = a->n_expert_used * a->n_tokens;
    if (a->M == 0 || nslices == 0) return 0;
    const int64_t kp = (a->K + 7) & ~(int64_t)7, xld = a->x_ld ? a->x_ld : a->K;
    const int64_t rows = a->ne11 * a->n_tokens;
    void *xs = nullptr;
    hipStream_t st = (hipStream_t)stream;
    if (int rc = grow_scratch(s, (size_t)std::max<int64_t>(1, rows * kp) * 4, &xs, st)) return rc;
    if (kp > 0) {
        hipLaunchKernelGGL(k_act<1>, dim3(grid_for(kp, 2), (unsigned)rows), dim3(k_block), 0, st, a->x, xld, xld, xs,
                           (int64_t)1, a->K, kp, s->T.cvt16);
        LNSHIP_HIP(hipGetLastError());
    }
    mm_args32 m{(const uint32_t *)a->w, (const uint32_t *)xs, a->dst, a->K, kp, a->M, 1,
                1, a->n_expert_used, 1, 1, a->M, kp * a->M, a->M, a->M,
                a->ids, a->ids_ld ? a->ids_ld : a->n_expert_used, a->ne11, a->n_expert, s->index_err};
    const mm16_shape sh = mm_shape_x32(m.M, 1, nslices, kp, s->cus, 4);
    switch (sh.nc * 10 + sh.cg) {
        case 12: return launch_mm32<1, 2>(m, s->T, nslices, s->cus, st);
        case 14: return launch_mm32<1, 4>(m, s->T, nslices, s->cus, st);
        default: return launch_mm32<1, 1>(m, s->T, nslices, s->cus, st);
    }
}

uint64_t lnship16_mul_mat_id_draws(int mode, int64_t K, int64_t M, int64_t n_expert_used, int64_t n_tokens) {
    if (mode != LNSHIP_MONTE || K <= 0) return 0;
    return (uint64_t)n_expert_used * (uint64_t)n_tokens * (uint64_t)M * (uint64_t)(K - 1);
}

static int rms16_common(int mode, const float *src, const float *w, float *dst, int64_t ncols, int64_t nrows,
                        float eps, uint16_t monte_seed, const uint16_t *monte_state, uint64_t monte_offset,
                        void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (mode < 0 || mode > 3 || ncols < 0 || nrows < 0) return fail(LNSHIP_EINVAL, "rms_norm: bad argument%s");
    if (ncols == 0 || nrows == 0) return 0;
    if ((nrows + 63) / 64 > 2147483647) return fail(LNSHIP_ERANGE, "rms_norm: too many rows%s");
    hipStream_t st = (hipStream_t)stream;
    switch (mode) {
        case LNSHIP_BASE: return launch_rms16<LNSHIP_BASE>(src, w, dst, ncols, nrows, eps, monte_seed, monte_state,
                                                           monte_offset, s->T, s->cus, st);
        case LNSHIP_MONTE: return launch_rms16<LNSHIP_MONTE>(src, w, dst, ncols, nrows, eps, monte_seed, monte_state,
                                                             monte_offset, s->T, s->cus, st);
        case LNSHIP_LPVIP: return launch_rms16<LNSHIP_LPVIP>(src, w, dst, ncols, nrows, eps, monte_seed, monte_state,
                                                             monte_offset, s->T, s->cus, st);
        default: return launch_rms16<LNSHIP_SUM32>(src, w, dst, ncols, nrows, eps, monte_seed, monte_state,
                                                   monte_offset, s->T, s->cus, st);
    }
}

int lnship16_rms_norm(int mode, const float *src, float *dst, int64_t ncols, int64_t nrows, float eps,
                      uint16_t monte_seed, void *stream) {
    return rms16_common(mode, src, nullptr, dst, ncols, nrows, eps, monte_seed, nullptr, 0, stream);
}

int lnship16_rms_norm_state(int mode, const float *src, float *dst, int64_t ncols, int64_t nrows, float eps,
                            const uint16_t *monte_state, uint64_t monte_offset, void *stream) {
    if (!monte_state) return fail(LNSHIP_EINVAL, "rms_norm: null monte_state%s");
    return rms16_common(mode, src, nullptr, dst, ncols, nrows, eps, 0, monte_state, monte_offset, stream);
}

int lnship16_rms_norm_mul(int mode, const float *src, const float *w, float *dst, int64_t ncols, int64_t nrows,
                          float eps, uint16_t monte_seed, const uint16_t *monte_state, uint64_t monte_offset,
                          void *stream) {
    if (!w) return fail(LNSHIP_EINVAL, "rms_norm_mul: null weight row%s");
    return rms16_common(mode, src, w, dst, ncols, nrows, eps, monte_seed, monte_state, monte_offset, stream);
}

// added to the sums the sum32 kernels predict (k_mm16_rms's rms sum,
// k_attn16's soft_max total): lnship_test_predict_skew
static uint32_t g_predict_skew = 0;

int lnship_test_decode_width(int w) {
    const int prev = g_decode_w;
    if (w == 0 || w == 16) g_decode_w = w;
    return prev;
}

int lnship_test_predict_skew(int skew) {
    const int prev = (int)g_predict_skew;
    g_predict_skew = (uint32_t)skew;
    return prev;
}

int lnship16_rms_norm_mul_mat(int mode, const float *x, const float *norm_w, float eps, const void *w, float *dst,
                              int64_t K, int64_t M, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (mode != LNSHIP_SUM32)
        return fail(LNSHIP_EINVAL, "rms_norm_mul_mat: sum32 only (other modes: lnship16_rms_norm_mul, then "
                                   "lnship16_mul_mat)%s");
    if (!x || !norm_w || !w || !dst || K < 1 || M < 0) return fail(LNSHIP_EINVAL, "rms_norm_mul_mat: bad argument%s");
    if (M == 0) return 0;
    const int64_t kp = (K + 7) & ~(int64_t)7;
    constexpr int PF = 8;
    const int64_t lds = mm_xl_offset<LNSHIP_SUM32>() + 2 * (kp * 2) + k_xl_pad;
    if (lds > k_lds_bytes - 1024) return fail(LNSHIP_ERANGE, "rms_norm_mul_mat: row too long for LDS%s");
    if ((uint64_t)M * 16 * PF + (uint64_t)M * 16 > 0xffffffffu)
        return fail(LNSHIP_ERANGE, "rms_norm_mul_mat: weight rows too long for 32-bit block offsets%s");
    // 16-row chain waves while every workgroup still gets a CU of its own
    const bool narrow = narrow_mm(M * 4 / 3, s->cus);
    if (int rc = narrow ? set_lds(k_mm16_rms<PF, 16>, (int)lds) : set_lds(k_mm16_rms<PF>, (int)lds)) return rc;
    mm_args16 m{(const uint16_t *)w, nullptr, x, dst, K, kp, M, 1, K, K, 1, 1, 1, 1, M, kp * M, M, M, 0, nullptr, 0};
    m.norm = norm_w;
    m.eps = eps;
    m.skew = g_predict_skew;
    // the codes of 1 / K and of eps, as the device's conversion reads them
    m.rms_ik = host_cvt16(1.0f / (float)K);
    m.rms_eps = host_cvt16(eps);
    const int rows = narrow ? 3 * 16 : k_rms_mm_rows;
    const uint64_t wgs = (uint64_t)((M + rows - 1) / rows);
    if (wgs > 0x7fffffffu) return fail(LNSHIP_ERANGE, "rms_norm_mul_mat: grid too large%s");
    m.xcd_sh = xcd_shift(wgs, s->cus);
    if (narrow)
        hipLaunchKernelGGL((k_mm16_rms<PF, 16>), dim3((unsigned)(wgs << m.xcd_sh)), dim3(k_block), (int)lds,
                           (hipStream_t)stream, m, s->T);
    else
        hipLaunchKernelGGL(k_mm16_rms<PF>, dim3((unsigned)(wgs << m.xcd_sh)), dim3(k_block), (int)lds,
                           (hipStream_t)stream, m, s->T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

static int rms32_common(const float *src, const float *w, float *dst, int64_t ncols, int64_t nrows, float eps,
                        void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (ncols < 0 || nrows < 0) return fail(LNSHIP_EINVAL, "rms_norm: bad argument%s");
    if (ncols == 0 || nrows == 0) return 0;
    const int64_t rs = (ncols + 3) & ~(int64_t)3;
    const int rb = rows_per_block(k_lds_pos32, rs, 4, nrows, s->cus);
    if (rb < 1) return fail(LNSHIP_ERANGE, "rms_norm: row too long for LDS%s");
    const int lds = k_lds_pos32 + (int)(rb * rs * 4);
    if (int rc = set_lds(k_rms32, lds)) return rc;
    hipLaunchKernelGGL(k_rms32, dim3((unsigned)((nrows + rb - 1) / rb)), dim3(k_block), lds, (hipStream_t)stream, src,
                       w, dst, ncols, nrows, rb, eps, s->T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship32_rms_norm(const float *src, float *dst, int64_t ncols, int64_t nrows, float eps, void *stream) {
    return rms32_common(src, nullptr, dst, ncols, nrows, eps, stream);
}

int lnship32_rms_norm_mul(const float *src, const float *w, float *dst, int64_t ncols, int64_t nrows, float eps,
                          void *stream) {
    if (!w) return fail(LNSHIP_EINVAL, "rms_norm_mul: null weight row%s");
    return rms32_common(src, w, dst, ncols, nrows, eps, stream);
}



int lnship16_soft_max(int mode, const lnship_soft_max_args *a, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (mode < 0 || mode > 3) return fail(LNSHIP_EINVAL, "unknown summation mode%s");
    if (int rc = check_sm(a)) return rc;
    const int64_t nrows = a->src_ne[1] * a->src_ne[2] * a->src_ne[3];
    if (a->src_ne[0] == 0 || nrows == 0) return 0;
    sm_args m{a->src, a->mask, a->dst, a->src_ne[0], a->src_ne[1], a->src_ne[2], a->src_ne[3],
              a->mask_ne[0], a->mask_ne[1], a->mask_ne[2], a->mask_ne[3], a->scale, a->monte_seed, 0,
              a->monte_state, a->monte_offset};
    hipStream_t st = (hipStream_t)stream;
    switch (mode) {
        case LNSHIP_BASE: return launch_sm16<LNSHIP_BASE>(m, nrows, s->T, s->cus, st);
        case LNSHIP_MONTE: return launch_sm16<LNSHIP_MONTE>(m, nrows, s->T, s->cus, st);
        case LNSHIP_LPVIP: return launch_sm16<LNSHIP_LPVIP>(m, nrows, s->T, s->cus, st);
        default: return launch_sm16<LNSHIP_SUM32>(m, nrows, s->T, s->cus, st);
    }
}

// the arguments of an LNS16 decode attention, checked before any device call
// (need_q: q is read; the fused rope forms it instead; monte: the caller
// passes the three nodes' Monte starts)
static int attn16_check(int mode, const lnship_attn_args *a, bool need_q, bool monte = false) {
    if (!a) return fail(LNSHIP_EINVAL, "attn_decode: null args%s");
    if (mode == LNSHIP_MONTE && !monte)
        return fail(LNSHIP_EINVAL, "attn_decode: Monte draws run across the three nodes in graph order: run them, "
                                   "or pass their starts to lnship16_attn_decode_seqs%s");
    if (mode < 0 || mode > 3) return fail(LNSHIP_EINVAL, "unknown summation mode%s");
    if ((need_q && !a->q) || !a->k_cache || !a->v_cache || !a->dst || a->n_head <= 0 || a->n_head_kv <= 0 ||
        a->n_head % a->n_head_kv || a->head_dim <= 0 || a->n_kv <= 0 || a->cache_m < a->n_kv ||
        a->head_dim > 4096 || a->n_head > 65535)
        return fail(LNSHIP_EINVAL, "attn_decode: bad argument%s");
    if (a->n_kv > lnship_max_row(8, mode)) return fail(LNSHIP_ERANGE, "attn_decode: n_kv too long for LDS%s");
    // the limit above holds for head_dim <= 256; wider heads need more LDS
    if ((int64_t)attn16_lds_mode(mode, a->head_dim, a->n_kv) > k_lds_bytes - k_lds_static)
        return fail(LNSHIP_ERANGE, "attn_decode: head_dim x n_kv too large for LDS%s");
    return 0;
}

static int attn16_launch(int mode, const attn_args &m, int64_t nh, const dev_tables &T, hipStream_t st) {
    switch (mode) {
        case LNSHIP_BASE: return launch_attn16<LNSHIP_BASE>(m, nh, T, st);
        case LNSHIP_MONTE: return launch_attn16<LNSHIP_MONTE>(m, nh, T, st);
        case LNSHIP_LPVIP: return launch_attn16<LNSHIP_LPVIP>(m, nh, T, st);
        default: return launch_attn16<LNSHIP_SUM32>(m, nh, T, st);
    }
}

int lnship16_attn_decode(int mode, const lnship_attn_args *a, void *stream) {
    // arguments and sizes first: they need no device
    if (int rc = attn16_check(mode, a, true)) return rc;
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    attn_args m{a->q, (const uint16_t *)a->k_cache, (const uint16_t *)a->v_cache, a->cache_m * 8, a->k_slice,
                      a->head_dim * 8, a->v_slice,
                      a->mask, a->scale, a->dst, (int)a->head_dim, (int)a->n_kv, (int)(a->n_head / a->n_head_kv),
                      g_predict_skew};
    m.nh = (int)a->n_head;
    m.nhkv = (int)a->n_head_kv;
    m.nseq = 1;
    return attn16_launch(mode, m, a->n_head, s->T, (hipStream_t)stream);
}

int lnship16_attn_decode_seqs(int mode, const lnship_attn_args *a, const lnship_attn_seqs *q, void *stream) {
    // arguments and sizes first: they need no device
    if (int rc = attn16_check(mode, a, true, true)) return rc;
    if (!q || q->n_seq <= 0 || a->n_head * q->n_seq > 0x7fffff)
        return fail(LNSHIP_EINVAL, "attn_decode_seqs: bad sequence count%s");
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    attn_args m{a->q, (const uint16_t *)a->k_cache, (const uint16_t *)a->v_cache, a->cache_m * 8, a->k_slice,
                a->head_dim * 8, a->v_slice,
                a->mask, a->scale, a->dst, (int)a->head_dim, (int)a->n_kv, (int)(a->n_head / a->n_head_kv),
                g_predict_skew};
    m.nh = (int)a->n_head;
    m.nhkv = (int)a->n_head_kv;
    m.nseq = (int)q->n_seq;
    for (int i = 0; i < 3; i++) {
        m.mseed[i] = q->monte_seed[i];
        m.moff[i] = q->monte_offset[i];
    }
    m.mstate = q->monte_state;
    return attn16_launch(mode, m, a->n_head * q->n_seq, s->T, (hipStream_t)stream);
}

// The store arguments of a rope-fused attention over n_seq sequences: the
// same heads and caches as the attention's, one token per sequence (row s
// of qkv, qkv_ld floats apart), no seq map: sequence s's cells lie at
// s n_head_kv k_slice and s n_head_kv v_slice, where the attention reads
// them, so seq_stride must say so when there is more than one
static bool rope_attn_store_ok(const lnship_qkv_store_args *q, const lnship_attn_args *a, int64_t n_seq) {
    return q && q->qkv && q->pos && q->cos_sin && q->ntok == n_seq && !q->seq && q->n_head == a->n_head &&
           q->n_head_kv == a->n_head_kv && q->head_dim == a->head_dim && q->head_dim % 8 == 0 &&
           q->rope_n_dims > 0 && q->rope_n_dims % 2 == 0 && q->rope_n_dims <= q->head_dim &&
           q->qkv_ld >= (q->n_head + 2 * q->n_head_kv) * q->head_dim && q->k_cache == a->k_cache &&
           q->v_cache == a->v_cache && q->cache_m == a->cache_m && q->k_slice == a->k_slice &&
           q->v_slice == a->v_slice &&
           (n_seq == 1 || (q->seq_stride == a->n_head_kv * a->k_slice && q->seq_stride == a->n_head_kv * a->v_slice));
}

static attn_args rope_attn_args(const lnship_qkv_store_args *q, const lnship_attn_args *a, const device_state *s) {
    attn_args m{nullptr, (const uint16_t *)a->k_cache, (const uint16_t *)a->v_cache, a->cache_m * 8,
                a->k_slice, a->head_dim * 8, a->v_slice,
                a->mask, a->scale, a->dst, (int)a->head_dim, (int)a->n_kv, (int)(a->n_head / a->n_head_kv),
                g_predict_skew, q->qkv, q->pos, q->cos_sin, q->rope_n_dims, (int)a->n_head,
                (int)a->n_head_kv, s->index_err, 1};
    m.qld = q->qkv_ld;
    return m;
}

int lnship16_rope_attn_decode(int mode, const lnship_qkv_store_args *q, const lnship_attn_args *a, void *stream) {
    // arguments and sizes first: they need no device
    if (int rc = attn16_check(mode, a, false)) return rc;
    if (!rope_attn_store_ok(q, a, 1))
        return fail(LNSHIP_EINVAL, "rope_attn_decode: the store arguments do not match the attention's%s");
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    return attn16_launch(mode, rope_attn_args(q, a, s), a->n_head, s->T, (hipStream_t)stream);
}

int lnship16_rope_attn_decode_seqs(int mode, const lnship_qkv_store_args *q, const lnship_attn_args *a,
                                   const lnship_attn_seqs *sq, void *stream) {
    // arguments and sizes first: they need no device
    if (int rc = attn16_check(mode, a, false, true)) return rc;
    if (!sq || sq->n_seq <= 0 || a->n_head * sq->n_seq > 0x7fffff)
        return fail(LNSHIP_EINVAL, "rope_attn_decode_seqs: bad sequence count%s");
    if (!rope_attn_store_ok(q, a, sq->n_seq))
        return fail(LNSHIP_EINVAL, "rope_attn_decode_seqs: the store arguments do not match the attention's%s");
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    attn_args m = rope_attn_args(q, a, s);
    m.nseq = (int)sq->n_seq;
    for (int i = 0; i < 3; i++) {
        m.mseed[i] = sq->monte_seed[i];
        m.moff[i] = sq->monte_offset[i];
    }
    m.mstate = sq->monte_state;
    return attn16_launch(mode, m, a->n_head * sq->n_seq, s->T, (hipStream_t)stream);
}

int lnship32_attn_decode(const lnship_attn_args *a, void *stream) {
    // arguments and sizes first: they need no device
    if (!a) return fail(LNSHIP_EINVAL, "attn_decode: null args%s");
    if (!a->q || !a->k_cache || !a->v_cache || !a->dst || a->n_head <= 0 || a->n_head_kv <= 0 ||
        a->n_head % a->n_head_kv || a->head_dim <= 0 || a->n_kv <= 0 || a->cache_m < a->n_kv ||
        a->head_dim > 4096 || a->n_head > 65535)
        return fail(LNSHIP_EINVAL, "attn_decode: bad argument%s");
    if (attn32_lds(a->head_dim, a->n_kv) > k_lds_bytes - k_lds_static)
        return fail(LNSHIP_ERANGE, "attn_decode: head_dim x n_kv too large for LDS%s");
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    const attn32_args m{a->q, (const uint32_t *)a->k_cache, (const uint32_t *)a->v_cache, a->cache_m * 8, a->k_slice,
                        a->head_dim * 8, a->v_slice, a->mask, a->scale, a->dst, (int)a->head_dim, (int)a->n_kv,
                        (int)(a->n_head / a->n_head_kv)};
    const int lds = (int)attn32_lds(a->head_dim, a->n_kv);
    if (int rc = set_lds(k_attn32, lds)) return rc;
    hipLaunchKernelGGL(k_attn32, dim3(attn_grid(a->n_head)), dim3(k_block), lds, (hipStream_t)stream, m, s->T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship32_soft_max(const lnship_soft_max_args *a, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (int rc = check_sm(a)) return rc;
    const int64_t nrows = a->src_ne[1] * a->src_ne[2] * a->src_ne[3];
    if (a->src_ne[0] == 0 || nrows == 0) return 0;
    sm_args m{a->src, a->mask, a->dst, a->src_ne[0], a->src_ne[1], a->src_ne[2], a->src_ne[3],
              a->mask_ne[0], a->mask_ne[1], a->mask_ne[2], a->mask_ne[3], a->scale, 0, 0};
    const int64_t rs = (m.n + 3) & ~(int64_t)3;
    m.rb = rows_per_block(k_lds_tab32, rs, 4, nrows, s->cus);
    if (m.rb < 1) return fail(LNSHIP_ERANGE, "soft_max: row too long for LDS%s");
    const int lds = k_lds_tab32 + (int)(m.rb * rs * 4);
    if (int rc = set_lds(k_softmax32, lds)) return rc;
    hipLaunchKernelGGL(k_softmax32, dim3((unsigned)((nrows + m.rb - 1) / m.rb)), dim3(k_block), lds,
                       (hipStream_t)stream, m, s->T);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int64_t lnship_max_row(int which, int mode) {
    if (which == 2) return max_row(k_lds_pos32, 4);
    if (which == 3) return max_row(k_lds_tab32, 4);
    if (which == 7) return ((k_lds_bytes - k_lds_static - attn32_lds(256, 0)) / 8) & ~(int64_t)7;
    if (which == 5) {
        // lnship16_rms_norm_mul_mat: the tables, the x row and h (4 B per k)
        if (mode != LNSHIP_SUM32) return 0;
        return ((k_lds_bytes - 1024 - mm_xl_offset<LNSHIP_SUM32>() - k_xl_pad) / 4) & ~(int64_t)7;
    }
    if (which == 6) {
        // lnship16_swiglu_mul_mat: one activation row in LDS beside the tables
        if (mode < 0 || mode > 3 || mode == LNSHIP_MONTE) return 0;
        return ((k_lds_bytes - 1024 - mm16_tables_bytes(mode) - k_xl_pad) / 2) & ~(int64_t)7;
    }
    if (which == 4 || which == 8) {
        switch (mode) {
            case LNSHIP_BASE: return max_attn_kv<LNSHIP_BASE>();
            case LNSHIP_MONTE: return which == 8 ? max_attn_kv<LNSHIP_MONTE>() : 0;
            case LNSHIP_LPVIP: return max_attn_kv<LNSHIP_LPVIP>();
            case LNSHIP_SUM32: return max_attn_kv<LNSHIP_SUM32>();
            default: return 0;
        }
    }
    if (which != 0 && which != 1) return 0;
    switch (mode) {
        case LNSHIP_BASE: return max_row(row_tables_bytes<LNSHIP_BASE>(), 2);
        case LNSHIP_MONTE: return max_row(row_tables_bytes<LNSHIP_MONTE>(), 2);
        case LNSHIP_LPVIP: return max_row(row_tables_bytes<LNSHIP_LPVIP>(), 2);
        case LNSHIP_SUM32: return max_row(row_tables_bytes<LNSHIP_SUM32>(), 2);
        default: return 0;
    }
}



int lnship16_add(const float *a, const float *b, int64_t n, int64_t nb, float *dst, void *stream) {
    return binary_common<16, 0>(a, b, n, nb, dst, stream);
}
int lnship16_mul(const float *a, const float *b, int64_t n, int64_t nb, float *dst, void *stream) {
    return binary_common<16, 1>(a, b, n, nb, dst, stream);
}
int lnship32_add(const float *a, const float *b, int64_t n, int64_t nb, float *dst, void *stream) {
    return binary_common<32, 0>(a, b, n, nb, dst, stream);
}
int lnship32_mul(const float *a, const float *b, int64_t n, int64_t nb, float *dst, void *stream) {
    return binary_common<32, 1>(a, b, n, nb, dst, stream);
}
int lnship16_scale(const float *src, float *dst, int64_t n, float s, float b, void *stream) {
    return scale_common<16>(src, dst, n, s, b, stream);
}
int lnship32_scale(const float *src, float *dst, int64_t n, float s, float b, void *stream) {
    return scale_common<32>(src, dst, n, s, b, stream);
}
int lnship16_swiglu(const float *gate, int64_t gate_ld, const float *up, int64_t up_ld, float *dst, int64_t ncols,
                    int64_t nrows, void *stream) {
    return swiglu_common<16>(gate, gate_ld, up, up_ld, dst, ncols, nrows, stream);
}
int lnship32_swiglu(const float *gate, int64_t gate_ld, const float *up, int64_t up_ld, float *dst, int64_t ncols,
                    int64_t nrows, void *stream) {
    return swiglu_common<32>(gate, gate_ld, up, up_ld, dst, ncols, nrows, stream);
}

int lnship16_get_rows_packed(const uint16_t *w, int64_t K, int64_t M, const int32_t *rows, int64_t nrows, float *dst,
                             void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (K < 0 || M <= 0 || nrows < 0) return fail(LNSHIP_EINVAL, "get_rows: bad shape%s");
    if (K == 0 || nrows == 0) return 0;
    hipLaunchKernelGGL(k_get_rows_packed, dim3(grid_for(nrows * K, 4)), dim3(k_block), 0, (hipStream_t)stream, w, K, M,
                       rows, nrows, dst, s->T.rev16);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}



int lnship16_rope(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                  int n_dims, int neox, const float *cos_sin, float *dst, void *stream) {
    return rope_common<16>(x, x_ld, pos, ntok, nhead, ne0, n_dims, neox, cos_sin, dst, stream);
}
int lnship32_rope(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                  int n_dims, int neox, const float *cos_sin, float *dst, void *stream) {
    return rope_common<32>(x, x_ld, pos, ntok, nhead, ne0, n_dims, neox, cos_sin, dst, stream);
}
int lnship16_store_kv(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                      int rope_n_dims, const float *cos_sin, uint16_t *cache, int64_t cache_m, int64_t cache_slice,
                      int cache_transposed, const int32_t *seq, int64_t seq_stride, void *stream) {
    return store_kv_common<16>(x, x_ld, pos, ntok, nhead, ne0, rope_n_dims, cos_sin, cache, cache_m, cache_slice,
                               cache_transposed, seq, seq_stride, stream);
}
int lnship32_store_kv(const float *x, int64_t x_ld, const int32_t *pos, int64_t ntok, int64_t nhead, int64_t ne0,
                      int rope_n_dims, const float *cos_sin, uint32_t *cache, int64_t cache_m, int64_t cache_slice,
                      int cache_transposed, const int32_t *seq, int64_t seq_stride, void *stream) {
    return store_kv_common<32>(x, x_ld, pos, ntok, nhead, ne0, rope_n_dims, cos_sin, cache, cache_m, cache_slice,
                               cache_transposed, seq, seq_stride, stream);
}
int lnship16_rope_store_kv(const lnship_qkv_store_args *a, void *stream) { return rope_store_kv_common<16>(a, stream); }
int lnship32_rope_store_kv(const lnship_qkv_store_args *a, void *stream) { return rope_store_kv_common<32>(a, stream); }

static bool strided_ok(const int64_t *ne, const int64_t *nb, strided4 &g) {
    if (!ne || !nb) return false;
    for (int d = 0; d < 4; d++) {
        if (ne[d] < 0 || nb[d] < 0) return false;
        g.ne[d] = ne[d];
        g.nb[d] = nb[d];
    }
    return true;
}

int lnship_gather_f32(const void *src, int src_type, const int64_t ne[4], const int64_t nb[4], float *dst,
                      void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    strided4 g;
    if (!strided_ok(ne, nb, g) || (src_type != 0 && src_type != 1)) return fail(LNSHIP_EINVAL, "gather: bad view%s");
    const int64_t n = ne[0] * ne[1] * ne[2] * ne[3];
    if (n == 0) return 0;
    if (src_type)
        hipLaunchKernelGGL(k_gather_f32<1>, dim3(grid_for(n, 4)), dim3(k_block), 0, (hipStream_t)stream,
                           (const char *)src, g, dst);
    else
        hipLaunchKernelGGL(k_gather_f32<0>, dim3(grid_for(n, 4)), dim3(k_block), 0, (hipStream_t)stream,
                           (const char *)src, g, dst);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship_scatter_f32(const float *src, void *dst, const int64_t ne[4], const int64_t nb[4], void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    strided4 g;
    if (!strided_ok(ne, nb, g)) return fail(LNSHIP_EINVAL, "scatter: bad view%s");
    const int64_t n = ne[0] * ne[1] * ne[2] * ne[3];
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_scatter_f32, dim3(grid_for(n, 4)), dim3(k_block), 0, (hipStream_t)stream, src, (char *)dst,
                       g);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship_copy(const void *src, int src_type, const int64_t src_ne[4], const int64_t src_nb[4], void *dst,
                int dst_type, const int64_t dst_ne[4], const int64_t dst_nb[4], void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    strided4 gs, gd;
    if (!strided_ok(src_ne, src_nb, gs) || !strided_ok(dst_ne, dst_nb, gd) || (src_type | dst_type) & ~1)
        return fail(LNSHIP_EINVAL, "copy: bad view%s");
    const int64_t n = gs.ne[0] * gs.ne[1] * gs.ne[2] * gs.ne[3];
    if (n != gd.ne[0] * gd.ne[1] * gd.ne[2] * gd.ne[3]) return fail(LNSHIP_EINVAL, "copy: element counts differ%s");
    if (n == 0) return 0;
    const dim3 g(grid_for(n, 4));
    hipStream_t st = (hipStream_t)stream;
    const char *x = (const char *)src;
    char *y = (char *)dst;
    switch (src_type * 2 + dst_type) {
        case 0: hipLaunchKernelGGL((k_copy<0, 0>), g, dim3(k_block), 0, st, x, gs, y, gd); break;
        case 1: hipLaunchKernelGGL((k_copy<0, 1>), g, dim3(k_block), 0, st, x, gs, y, gd); break;
        case 2: hipLaunchKernelGGL((k_copy<1, 0>), g, dim3(k_block), 0, st, x, gs, y, gd); break;
        default: hipLaunchKernelGGL((k_copy<1, 1>), g, dim3(k_block), 0, st, x, gs, y, gd); break;
    }
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

static bool ids_ok(const int64_t *ne, const int64_t *nb, ids3 &g) {
    if (!ne || !nb) return false;
    for (int d = 0; d < 3; d++) {
        if (ne[d] < 0 || nb[d] < 0) return false;
        g.ne[d] = ne[d];
        g.nb[d] = nb[d];
    }
    return true;
}

int lnship_get_rows(const void *src, int src_type, const int64_t src_ne[4], const int64_t src_nb[4],
                    const int32_t *ids, const int64_t ids_ne[3], const int64_t ids_nb[3], float *dst,
                    const int64_t dst_nb[4], void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    strided4 gs, gd;
    ids3 gi;
    if (!strided_ok(src_ne, src_nb, gs) || !ids_ok(ids_ne, ids_nb, gi) || (src_type & ~1))
        return fail(LNSHIP_EINVAL, "get_rows: bad view%s");
    const int64_t dne[4] = {src_ne[0], ids_ne[0], ids_ne[1], ids_ne[2]};
    if (!strided_ok(dne, dst_nb, gd)) return fail(LNSHIP_EINVAL, "get_rows: bad destination view%s");
    if (src_ne[2] != ids_ne[1] || src_ne[3] != ids_ne[2])
        return fail(LNSHIP_EINVAL, "get_rows: index slices do not match the source's%s");
    const int64_t n = dne[0] * dne[1] * dne[2] * dne[3];
    if (n == 0) return 0;
    const dim3 g(grid_for(n, 4));
    if (src_type)
        hipLaunchKernelGGL(k_get_rows<1>, g, dim3(k_block), 0, (hipStream_t)stream, (const char *)src, gs,
                           (const char *)ids, gi, dst, gd, s->index_err);
    else
        hipLaunchKernelGGL(k_get_rows<0>, g, dim3(k_block), 0, (hipStream_t)stream, (const char *)src, gs,
                           (const char *)ids, gi, dst, gd, s->index_err);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship_set_rows(const float *src, const int64_t src_ne[4], const int64_t src_nb[4], const void *ids,
                    int ids_i64, const int64_t ids_ne[3], const int64_t ids_nb[3], void *dst, int dst_type,
                    const int64_t dst_ne[4], const int64_t dst_nb[4], void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    strided4 gs, gd;
    ids3 gi;
    if (!strided_ok(src_ne, src_nb, gs) || !strided_ok(dst_ne, dst_nb, gd) || !ids_ok(ids_ne, ids_nb, gi) ||
        (dst_type & ~1) || (ids_i64 & ~1))
        return fail(LNSHIP_EINVAL, "set_rows: bad view%s");
    if (src_ne[0] != dst_ne[0] || src_ne[2] != dst_ne[2] || src_ne[3] != dst_ne[3] || src_ne[1] != ids_ne[0])
        return fail(LNSHIP_EINVAL, "set_rows: shapes do not match%s");
    const int64_t n = src_ne[0] * src_ne[1] * src_ne[2] * src_ne[3];
    if (n == 0) return 0;
    if (ids_ne[1] <= 0 || ids_ne[2] <= 0 || src_ne[2] % ids_ne[1] || src_ne[3] % ids_ne[2])
        return fail(LNSHIP_EINVAL, "set_rows: index slices do not broadcast%s");
    const dim3 g(grid_for(n, 4));
    if (dst_type)
        hipLaunchKernelGGL(k_set_rows<1>, g, dim3(k_block), 0, (hipStream_t)stream, (const char *)src, gs,
                           (const char *)ids, gi, ids_i64, (char *)dst, gd, s->index_err);
    else
        hipLaunchKernelGGL(k_set_rows<0>, g, dim3(k_block), 0, (hipStream_t)stream, (const char *)src, gs,
                           (const char *)ids, gi, ids_i64, (char *)dst, gd, s->index_err);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship_lpvip_db_range(uint32_t d0, uint32_t n, int32_t *out, void *stream) {
    // arguments first: they need no device
    if (!out) return fail(LNSHIP_EINVAL, "lpvip_db_range: null output%s");
    // d = 0 is exact cancellation, which the adder handles before db
    if (d0 == 0 || (uint64_t)d0 + n > 0x100000000ull) return fail(LNSHIP_EINVAL, "lpvip_db_range: d outside [1, 2^32)%s");
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_lpvip_db_range, dim3(grid_for(n, 4)), dim3(k_block), 0, (hipStream_t)stream, d0, n, out,
                       s->T.lpdb);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship32_add_lds(int form, const uint32_t *x, const uint32_t *y, uint32_t *out, int64_t n, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    if (form < 0 || form > 3 || n < 0) return fail(LNSHIP_EINVAL, "add_lds: bad argument%s");
    if (n == 0) return 0;
    if (!x || !y || !out) return fail(LNSHIP_EINVAL, "add_lds: null pointer%s");
    // one staging of the tables per workgroup: a grid of one workgroup per CU
    const dim3 g((unsigned)std::min<int64_t>((n + k_block - 1) / k_block, std::max(s->cus, 1)));
    hipStream_t st = (hipStream_t)stream;
    switch (form) {
        case 0:
            if (int rc = set_lds(k_x32_add_lds<0>, k_lds_tab32)) return rc;
            hipLaunchKernelGGL(k_x32_add_lds<0>, g, dim3(k_block), k_lds_tab32, st, x, y, out, n, s->T);
            break;
        case 1:
            if (int rc = set_lds(k_x32_add_lds<1>, k_lds_tab32)) return rc;
            hipLaunchKernelGGL(k_x32_add_lds<1>, g, dim3(k_block), k_lds_tab32, st, x, y, out, n, s->T);
            break;
        case 2:
            if (int rc = set_lds(k_x32_add_lds<2>, k_lds_tab32)) return rc;
            hipLaunchKernelGGL(k_x32_add_lds<2>, g, dim3(k_block), k_lds_tab32, st, x, y, out, n, s->T);
            break;
        default:
            if (int rc = set_lds(k_x32_add_lds<3>, k_lds_pos32)) return rc;
            hipLaunchKernelGGL(k_x32_add_lds<3>, g, dim3(k_block), k_lds_pos32, st, x, y, out, n, s->T);
    }
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

int lnship_index_error(int64_t *bad_index, void *stream) {
    device_state *s = state();
    if (!s) return LNSHIP_ENOINIT;
    LNSHIP_HIP(hipStreamSynchronize((hipStream_t)stream));
    unsigned long long e[2];
    LNSHIP_HIP(hipMemcpy(e, s->index_err, sizeof e, hipMemcpyDeviceToHost));
    if (!e[0]) return 0;
    const unsigned long long zero[2] = {0, 0};
    LNSHIP_HIP(hipMemcpy(s->index_err, zero, sizeof zero, hipMemcpyHostToDevice));
    if (bad_index) *bad_index = (int64_t)e[1];
    return 1;
}

int lnship_rope_table(float freq_base, int n_dims, int64_t n_pos, float *out) {
    if (n_dims <= 0 || n_dims % 2 || n_pos < 0 || !out) return fail(LNSHIP_EINVAL, "rope_table: bad argument%s");
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    const int half = n_dims / 2;
    for (int64_t p = 0; p < n_pos; p++) {
        float t = (float)p;
        for (int j = 0; j < half; j++) {
            out[(p * half + j) * 2 + 0] = cosf(t);
            out[(p * half + j) * 2 + 1] = sinf(t);
            t *= theta_scale;
        }
    }
    return 0;
}

int lnship_causal_mask(const int32_t *pos, int64_t ntok, int64_t n_kv, float *mask, void *stream) {
    if (ntok < 0 || n_kv < 0) return fail(LNSHIP_EINVAL, "causal_mask: bad shape%s");
    if (ntok == 0 || n_kv == 0) return 0;
    hipLaunchKernelGGL(k_causal_mask, dim3(grid_for(ntok * n_kv, 4)), dim3(k_block), 0, (hipStream_t)stream, pos, ntok,
                       n_kv, mask);
    LNSHIP_HIP(hipGetLastError());
    return 0;
}

}  // extern "C"
