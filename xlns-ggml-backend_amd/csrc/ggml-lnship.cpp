// LNSHIP16 / LNSHIP32: the lnship HIP kernels as ggml backends.
//
// What ggml sees is what the reference's LNSCUDA16 / LNSCUDA32 backends show
// it (lns-backend/cuda/ggml-lns-cuda.cpp, common/lns-backend-framework.h):
//   - a registry per device (get_name, get_device_count, get_device,
//     get_proc_address), api_version GGML_BACKEND_API_VERSION;
//   - an ACCEL device on the CPU buffer type (host memory), caps async=false,
//     host_buffer=false, buffer_from_host_ptr=true, events=false; its
//     description carries "sum=<mode>" for xlns16 (scripts parse it);
//   - a backend whose only non-null slots are get_name, free, graph_compute;
//   - supports_op = this file's predicates, filtered by GGML_LNS_BACKEND,
//     LNS_DISABLE_OPS, LNS_ENABLE_OPS, logged by LNS_OP_AUDIT; offload_op
//     = supports_op, so the scheduler prefers this device over the CPU
//     backend on the same host buffers.
// Inside graph_compute each claimed node uploads its F32 inputs into HBM,
// runs the lnship C ABI and downloads its result before the next node (any
// backend may read it).  Weights (GGML_BACKEND_BUFFER_USAGE_WEIGHTS) are
// packed into the k8-interleaved LNS layout once and stay in HBM, keyed by
// (data, type, ne, nb) as llama.cpp never rewrites a weight in place.
//
// ggml's op and type enums are never compared as numbers: nodes are matched
// by ggml_op_name / ggml_op_desc / ggml_type_name (see ggml_abi.h).
//
// Threading: graph_compute is single-threaded per backend instance and may
// run on any host thread (the device is re-selected on every call).  The
// kernels' activation scratch is per device, so two instances must not run
// graph_compute on the same GPU at the same time.

#include "ggml_abi.h"
#include "ggml-lnship.h"
#include "lnship.h"

#include <hip/hip_runtime.h>

#include <dlfcn.h>
#include <fnmatch.h>
#include <strings.h>

#include <algorithm>
#include <array>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <tuple>
#include <vector>

namespace lnship_ggml {

// ============================================================ errors

[[noreturn]] static void die(const char *fmt, ...) {
    std::fprintf(stderr, "ggml-lnship: ");
    va_list ap;
    va_start(ap, fmt);
    std::vfprintf(stderr, fmt, ap);
    va_end(ap);
    std::fputc('\n', stderr);
    std::fflush(stderr);
    std::abort();
}

static void hip_ok(hipError_t e, const char *what) {
    if (e != hipSuccess) die("%s: %s", what, hipGetErrorString(e));
}

static void lib_ok(int rc, const char *what) {
    if (rc != 0) die("%s returned %d: %s", what, rc, lnship_last_error());
}

// ============================================================ environment

static bool env_flag(const char *name) {
    const char *v = std::getenv(name);
    return v && v[0] && std::strcmp(v, "0") != 0;
}

// "a, b,,c" -> {"a", "b", "c"}
static std::vector<std::string> split_list(const std::string &s) {
    std::vector<std::string> out;
    size_t i = 0;
    while (i <= s.size()) {
        size_t j = s.find(',', i);
        if (j == std::string::npos) j = s.size();
        const size_t a = s.find_first_not_of(" \t", i);
        if (a != std::string::npos && a < j) {
            const size_t b = s.find_last_not_of(" \t", j - 1);
            out.push_back(s.substr(a, b - a + 1));
        }
        i = j + 1;
    }
    return out;
}

static std::vector<std::string> env_list(const char *name) {
    const char *v = std::getenv(name);
    return v ? split_list(v) : std::vector<std::string>();
}

// GGML_LNS_BACKEND: comma-separated aliases or device names, case-insensitive
// (common/lns-backend-config.h:60-140).  A GPU alias also selects the CPU LNS
// backend of the same format, so ops the GPU declines still run in LNS.
struct alias {
    const char *token;
    const char *devices;
};
static const alias k_aliases[] = {
    {"16", "LNS16"},
    {"32", "LNS32"},
    {"hip", "LNSHIP16,LNS16"},
    {"hip16", "LNSHIP16,LNS16"},
    {"hip32", "LNSHIP32,LNS32"},
    {"cuda", "LNSCUDA16,LNS16"},
    {"cuda16", "LNSCUDA16,LNS16"},
    {"cuda32", "LNSCUDA32,LNS32"},
};
static const char *const k_default_selection = "16";

static bool known_device(const std::string &name) {
    for (const alias &a : k_aliases)
        for (const std::string &d : split_list(a.devices))
            if (strcasecmp(d.c_str(), name.c_str()) == 0) return true;
    return false;
}

static std::vector<std::string> resolve_selection(const char *value) {
    const std::string spec = value && value[0] ? value : k_default_selection;
    std::vector<std::string> devs;
    for (const std::string &tok : split_list(spec)) {
        const alias *hit = nullptr;
        for (const alias &a : k_aliases)
            if (strcasecmp(a.token, tok.c_str()) == 0) hit = &a;
        if (hit) {
            for (const std::string &d : split_list(hit->devices)) devs.push_back(d);
        } else if (known_device(tok)) {
            devs.push_back(tok);
        } else {
            std::fprintf(stderr, "ggml-lnship: ignoring unknown GGML_LNS_BACKEND token '%s'\n", tok.c_str());
        }
    }
    return devs.empty() ? resolve_selection(k_default_selection) : devs;
}

static bool device_selected(const char *name) {
    static const std::vector<std::string> sel = resolve_selection(std::getenv("GGML_LNS_BACKEND"));
    for (const std::string &d : sel)
        if (strcasecmp(d.c_str(), name) == 0) return true;
    return false;
}

// LNS_DISABLE_OPS / LNS_ENABLE_OPS tokens (common/lns-backend-config.h:141-200):
// an op name or description (case-insensitive), "OP:pattern", a tensor-name
// substring or glob, or "<pattern" for the name of src[1].
static bool name_matches(const char *name, const std::string &pat) {
    if (!name || !name[0] || pat.empty()) return false;
    if (pat.find_first_of("*?[") != std::string::npos) return fnmatch(pat.c_str(), name, 0) == 0;
    return std::strstr(name, pat.c_str()) != nullptr;
}

static bool op_matches(const ggml_tensor *op, const std::string &tok) {
    const char *on = ggml_op_name(op->op), *od = ggml_op_desc(op);
    if (strcasecmp(tok.c_str(), on) == 0 || strcasecmp(tok.c_str(), od) == 0) return true;
    std::string pat = tok;
    const size_t colon = tok.find(':');
    if (colon != std::string::npos) {
        const std::string want = tok.substr(0, colon);
        if (strcasecmp(want.c_str(), on) != 0 && strcasecmp(want.c_str(), od) != 0) return false;
        pat = tok.substr(colon + 1);
    }
    if (!pat.empty() && pat[0] == '<') return op->src[1] && name_matches(op->src[1]->name, pat.substr(1));
    return name_matches(op->name, pat);
}

static bool any_match(const ggml_tensor *op, const std::vector<std::string> &toks) {
    for (const std::string &t : toks)
        if (op_matches(op, t)) return true;
    return false;
}

static bool op_disabled(const ggml_tensor *op) {
    static const std::vector<std::string> off = env_list("LNS_DISABLE_OPS");
    static const bool have_on = std::getenv("LNS_ENABLE_OPS") != nullptr;
    static const std::vector<std::string> on = env_list("LNS_ENABLE_OPS");
    if (have_on && !any_match(op, on)) return true;
    return any_match(op, off);
}

// One JSON record per supports_op query (common/lns-backend-config.h:205-240).
static void audit(const char *backend, const char *extra, const ggml_tensor *op, bool ok, const char *reason) {
    static const bool on = env_flag("LNS_OP_AUDIT");
    if (!on) return;
    auto tn = [](const ggml_tensor *t) { return t ? ggml_type_name(t->type) : "null"; };
    std::fprintf(stderr,
                 "{\"event\":\"lns_supports_op\",\"backend\":\"%s\",%s\"op\":\"%s\",\"desc\":\"%s\","
                 "\"supported\":%s,\"dst_type\":\"%s\",\"src_types\":[\"%s\",\"%s\",\"%s\",\"%s\"],"
                 "\"shape\":[%lld,%lld,%lld,%lld],\"reason\":\"%s\"}\n",
                 backend, extra, ggml_op_name(op->op), ggml_op_desc(op), ok ? "true" : "false",
                 ggml_type_name(op->type), tn(op->src[0]), tn(op->src[1]), tn(op->src[2]), tn(op->src[3]),
                 (long long)op->ne[0], (long long)op->ne[1], (long long)op->ne[2], (long long)op->ne[3], reason);
}

// GGML_LNS16_SUM: the xlns16 summation mode (the reference fixes it at build
// time, common/lns-common.cmake:24-28; here it is read once at run time).
static int sum_mode() {
    static const int mode = []() {
        const char *v = std::getenv("GGML_LNS16_SUM");
        if (!v || !v[0] || !std::strcmp(v, "base")) return (int)LNSHIP_BASE;
        if (!std::strcmp(v, "monte")) return (int)LNSHIP_MONTE;
        if (!std::strcmp(v, "lpvip")) return (int)LNSHIP_LPVIP;
        if (!std::strcmp(v, "sum32")) return (int)LNSHIP_SUM32;
        die("GGML_LNS16_SUM must be one of base, monte, lpvip, sum32 (got '%s')", v);
    }();
    // GGML_LNS16_MONTE_BYLPVIP (the reference's second Monte build,
    // src/lns-ops.cpp:86-98): its library source, xlns16monte_bylpvip.cpp, is
    // not available, so a Monte run that asks for it stops here rather than
    // running the other Monte adder under its name
    static const bool checked = []() {
        const char *b = std::getenv("GGML_LNS16_MONTE_BYLPVIP");
        if (mode == LNSHIP_MONTE && b && b[0] && std::strcmp(b, "0") && strcasecmp(b, "OFF") && strcasecmp(b, "false"))
            die("GGML_LNS16_MONTE_BYLPVIP=%s: monte=bylpvip is not available in this backend (only monte=pure16)", b);
        return true;
    }();
    (void)checked;
    return mode;
}

// LNS16_SUM_POLICY (cuda/lns-cuda-context.cpp:221-269): comma-separated
// "selector=mode" rules, selectors as LNS_DISABLE_OPS's; the first rule that
// matches a node sets its summation mode.  base, lpvip and sum32 are always
// available (every mode is in this library, as the reference's
// GGML_LNSCUDA16_MIXED build); monte only as GGML_LNS16_SUM itself, since the
// Monte state belongs to that mode.  A malformed rule aborts.
static const std::vector<std::pair<std::string, int>> &sum_policy() {
    static const std::vector<std::pair<std::string, int>> rules = []() {
        std::vector<std::pair<std::string, int>> r;
        const char *env = std::getenv("LNS16_SUM_POLICY");
        if (!env) return r;
        for (const std::string &rule : split_list(env)) {
            const size_t eq = rule.rfind('=');
            if (eq == std::string::npos) die("LNS16_SUM_POLICY rule '%s' is not selector=mode", rule.c_str());
            const std::string m = rule.substr(eq + 1);
            int mode = -1;
            if (m == "base") mode = LNSHIP_BASE;
            else if (m == "lpvip") mode = LNSHIP_LPVIP;
            else if (m == "sum32") mode = LNSHIP_SUM32;
            else if (m == "monte" && sum_mode() == LNSHIP_MONTE) mode = LNSHIP_MONTE;
            if (mode < 0)
                die("LNS16_SUM_POLICY mode '%s' is not available (base|lpvip|sum32; monte only as GGML_LNS16_SUM)",
                    m.c_str());
            r.emplace_back(rule.substr(0, eq), mode);
        }
        std::fprintf(stderr, "ggml-lnship: LNSHIP16 LNS16_SUM_POLICY with %zu rules (default sum=%s)\n", r.size(),
                     sum_mode() == LNSHIP_MONTE ? "monte"
                     : sum_mode() == LNSHIP_LPVIP ? "lpvip"
                     : sum_mode() == LNSHIP_SUM32 ? "sum32"
                                                  : "base");
        return r;
    }();
    return rules;
}

// the summation mode of one xlns16 node
static int node_mode(const ggml_tensor *node) {
    for (const auto &rule : sum_policy())
        if (op_matches(node, rule.first)) return rule.second;
    return sum_mode();
}

static const char *mode_name(int m) {
    switch (m) {
        case LNSHIP_MONTE: return "monte";
        case LNSHIP_LPVIP: return "lpvip";
        case LNSHIP_SUM32: return "sum32";
        default: return "base";
    }
}

// GGML_LNS_HIP_DEVICE (default 0); -1 when that GPU does not exist or no HIP
// runtime is usable.
static int hip_device() {
    static const int dev = []() {
        const char *v = std::getenv("GGML_LNS_HIP_DEVICE");
        const int want = v ? std::atoi(v) : 0;
        int n = 0;
        if (hipGetDeviceCount(&n) != hipSuccess) {
            (void)hipGetLastError();
            return -1;
        }
        if (want < 0 || want >= n) {
            if (n > 0)
                std::fprintf(stderr, "ggml-lnship: GGML_LNS_HIP_DEVICE=%d, but there are %d GPU(s); LNSHIP disabled\n",
                             want, n);
            return -1;
        }
        return want;
    }();
    return dev;
}

// ============================================================ tensors

static bool type_is(const ggml_tensor *t, const char *name) {
    return t && std::strcmp(ggml_type_name(t->type), name) == 0;
}
static bool is_f32(const ggml_tensor *t) { return type_is(t, "f32"); }
static bool is_f16(const ggml_tensor *t) { return type_is(t, "f16"); }

static bool to_f32_possible(const ggml_tensor *t) {
    if (is_f32(t)) return true;
    const ggml_type_traits *tr = ggml_get_type_traits(t->type);
    return tr && tr->to_float;
}

static bool rows_contiguous(const ggml_tensor *t) { return t->nb[0] == ggml_type_size(t->type); }

static int64_t nelements(const ggml_tensor *t) { return t->ne[0] * t->ne[1] * t->ne[2] * t->ne[3]; }
static int64_t nrows(const ggml_tensor *t) { return t->ne[1] * t->ne[2] * t->ne[3]; }

// ggml_is_contiguous: dense in ggml element order (dimensions of size 1 may
// carry any stride)
static bool contiguous(const ggml_tensor *t) {
    size_t next = ggml_type_size(t->type);
    if (t->ne[0] != 1 && t->nb[0] != next) return false;
    next = next * (size_t)(t->ne[0] / ggml_blck_size(t->type));
    for (int i = 1; i < GGML_MAX_DIMS; i++) {
        if (t->ne[i] != 1) {
            if (t->nb[i] != next) return false;
            next *= (size_t)t->ne[i];
        }
    }
    return true;
}

static bool same_shape(const ggml_tensor *a, const ggml_tensor *b) {
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (a->ne[i] != b->ne[i]) return false;
    return true;
}

static bool can_repeat(const ggml_tensor *b, const ggml_tensor *a) {   // b broadcast over a
    for (int i = 0; i < GGML_MAX_DIMS; i++)
        if (b->ne[i] <= 0 || a->ne[i] % b->ne[i] != 0) return false;
    return true;
}

static float op_f32(const ggml_tensor *t, int i) {
    float v;
    std::memcpy(&v, &t->op_params[i], sizeof v);
    return v;
}
static int32_t op_i32(const ggml_tensor *t, int i) { return t->op_params[i]; }

static bool is_weight(const ggml_tensor *t) {
    return t->buffer && ggml_backend_buffer_get_usage(t->buffer) == GGML_BACKEND_BUFFER_USAGE_WEIGHTS;
}

// Rows of t as contiguous F32 in ggml element order (F32 copied, every other
// type through ggml's to_float).
static void gather_f32(const ggml_tensor *t, float *out) {
    const int64_t ne0 = t->ne[0];
    const size_t ts = ggml_type_size(t->type);
    const ggml_type_traits *tr = is_f32(t) ? nullptr : ggml_get_type_traits(t->type);
    const bool dense_rows = t->nb[0] == ts || (tr && tr->is_quantized);
    for (int64_t i3 = 0; i3 < t->ne[3]; i3++)
        for (int64_t i2 = 0; i2 < t->ne[2]; i2++)
            for (int64_t i1 = 0; i1 < t->ne[1]; i1++) {
                const char *row = (const char *)t->data + i1 * t->nb[1] + i2 * t->nb[2] + i3 * t->nb[3];
                float *o = out + ((i3 * t->ne[2] + i2) * t->ne[1] + i1) * ne0;
                if (dense_rows) {
                    if (!tr) std::memcpy(o, row, (size_t)ne0 * sizeof(float));
                    else tr->to_float(row, o, ne0);
                } else {
                    for (int64_t i = 0; i < ne0; i++) {
                        if (!tr) std::memcpy(o + i, row + i * t->nb[0], sizeof(float));
                        else tr->to_float(row + i * t->nb[0], o + i, 1);
                    }
                }
            }
}

static void scatter_f32(const float *in, ggml_tensor *t) {
    const int64_t ne0 = t->ne[0];
    for (int64_t i3 = 0; i3 < t->ne[3]; i3++)
        for (int64_t i2 = 0; i2 < t->ne[2]; i2++)
            for (int64_t i1 = 0; i1 < t->ne[1]; i1++) {
                char *row = (char *)t->data + i1 * t->nb[1] + i2 * t->nb[2] + i3 * t->nb[3];
                const float *s = in + ((i3 * t->ne[2] + i2) * t->ne[1] + i1) * ne0;
                for (int64_t i = 0; i < ne0; i++) std::memcpy(row + i * t->nb[0], s + i, sizeof(float));
            }
}

// ============================================================ op predicates

static bool on_device(const ggml_tensor *t);
static bool device_buffers();

enum class kind { view, mul_mat, mul_mat_id, rms_norm, soft_max, add, mul, swiglu, rope, scale, copy, get_rows,
                  set_rows, unary, glu, other };

static kind classify(const ggml_tensor *t) {
    const char *n = ggml_op_name(t->op);
    auto is = [n](const char *s) { return std::strcmp(n, s) == 0; };
    if (is("NONE") || is("RESHAPE") || is("VIEW") || is("PERMUTE") || is("TRANSPOSE")) return kind::view;
    if (is("MUL_MAT")) return kind::mul_mat;
    if (is("MUL_MAT_ID")) return kind::mul_mat_id;
    if (is("RMS_NORM")) return kind::rms_norm;
    if (is("SOFT_MAX")) return kind::soft_max;
    if (is("ADD")) return kind::add;
    if (is("MUL")) return kind::mul;
    if (is("ROPE")) return kind::rope;
    if (is("GLU")) return std::strcmp(ggml_op_desc(t), "SWIGLU") == 0 ? kind::swiglu : kind::glu;
    if (is("UNARY")) return kind::unary;
    if (is("SCALE")) return kind::scale;
    if (is("CPY") || is("CONT") || is("DUP")) return kind::copy;
    if (is("GET_ROWS")) return kind::get_rows;
    if (is("SET_ROWS")) return kind::set_rows;
    return kind::other;
}

struct verdict {
    bool ok;
    const char *reason;
};

// The node writes an F32 result of src[0]'s shape.
static verdict f32_result(const ggml_tensor *op, verdict v) {
    if (!v.ok) return v;
    if (!is_f32(op) || !same_shape(op, op->src[0])) return {false, "lnship_requires_f32_dst_of_src0_shape"};
    return v;
}

// common/lns-op-support.h:33-41 plus cuda/lns-cuda-ops.cpp:37-56
// GGML_TYPE_LNS16 weights (xlns16 codes, patches/ggml-core.patch:21-27) are
// taken as they are by the xlns16 backend, as row_to_xlns16 does
// (src/lns-ops.cpp:221-225); the reference's own predicate declines them,
// since the type has no to_float.
static bool lns16_codes(const ggml_tensor *t, bool w32) { return !w32 && type_is(t, "lns16"); }

static verdict check_mul_mat(const ggml_tensor *op, bool w32) {
    const ggml_tensor *a = op->src[0], *b = op->src[1];
    const bool codes = lns16_codes(a, w32);
    if (!is_f32(b) || !(codes || to_f32_possible(a))) return {false, "mul_mat_requires_src1_f32_and_convertible_src0"};
    if (codes && !contiguous(a)) return {false, "lnship_lns16_weights_require_contiguous"};
    if (on_device(a) && !is_f32(a) && !is_f16(a) && !codes) return {false, "lnship_device_src0_requires_f32_or_f16"};
    if (!rows_contiguous(a) || !rows_contiguous(b)) return {false, "mul_mat_requires_contiguous_rows"};
    if (!is_f32(op)) return {false, "lnship_mul_mat_requires_f32_dst"};
    if ((b->ne[1] + 3) / 4 > 65535 || b->ne[2] * b->ne[3] > 65535) return {false, "lnship_mul_mat_grid_too_large"};
    if (b->ne[2] % a->ne[2] != 0 || b->ne[3] % a->ne[3] != 0) return {false, "lnship_mul_mat_requires_whole_broadcast"};
    if (a->ne[0] > ((int64_t)1 << 30)) return {false, "lnship_mul_mat_k_too_large"};
    return {true, "lnship_mul_mat"};
}

// common/lns-op-support.h:43-50 plus the GEMV's limits (as check_mul_mat)
static verdict check_mul_mat_id(const ggml_tensor *op) {
    const ggml_tensor *a = op->src[0], *b = op->src[1], *ids = op->src[2];
    if (!b || !is_f32(b) || !ids || !type_is(ids, "i32") || !to_f32_possible(a))
        return {false, "mul_mat_id_requires_src1_f32_and_i32_ids_and_convertible_src0"};
    if (on_device(a) && !is_f32(a) && !is_f16(a)) return {false, "lnship_device_src0_requires_f32_or_f16"};
    if (!rows_contiguous(a) || !rows_contiguous(b)) return {false, "mul_mat_requires_contiguous_rows"};
    if (!is_f32(op)) return {false, "lnship_mul_mat_requires_f32_dst"};
    const int64_t neu = ids->ne[0], T = ids->ne[1];
    if (a->ne[3] != 1 || b->ne[3] != 1 || ids->ne[2] != 1 || ids->ne[3] != 1 || b->ne[0] != a->ne[0] ||
        b->ne[2] != T || b->ne[1] <= 0 || neu % b->ne[1] != 0 || op->ne[0] != a->ne[1] || op->ne[1] != neu ||
        op->ne[2] != T)
        return {false, "lnship_mul_mat_id_shape"};
    if (on_device(ids) && (ids->nb[0] != 4 || ids->nb[1] % 4 != 0))
        return {false, "lnship_mul_mat_id_requires_dense_device_ids"};
    if (neu * T > 65535) return {false, "lnship_mul_mat_id_too_many_slots"};
    if (a->ne[0] > ((int64_t)1 << 30)) return {false, "lnship_mul_mat_k_too_large"};
    return {true, "lnship_mul_mat_id"};
}

static verdict check_rms_norm(const ggml_tensor *op, bool w32) {
    verdict v = f32_result(op, {is_f32(op->src[0]), "unary_like_requires_src0_f32"});
    if (v.ok && op->src[0]->ne[0] > lnship_max_row(w32 ? 2 : 0, w32 ? 0 : node_mode(op))) return {false, "lnship_row_too_long"};
    return v;
}

// common/lns-op-support.h:126-140 plus cuda/lns-cuda-ops.cpp:181-190
static verdict check_soft_max(const ggml_tensor *op, bool w32) {
    const ggml_tensor *mask = op->src[1];
    if (!is_f32(op->src[0]) || (mask && !is_f32(mask))) return {false, "soft_max_requires_f32_src0_and_f32_mask"};
    if (op->src[2]) return {false, "soft_max_sinks_unsupported"};
    if (op_f32(op, 1) != 0.0f) return {false, "soft_max_alibi_unsupported"};
    verdict v = f32_result(op, {true, "soft_max_f32"});
    if (!v.ok) return v;
    if (mask && (mask->ne[0] < op->ne[0] || mask->ne[1] < op->ne[1]))
        return {false, "lnship_soft_max_mask_smaller_than_src0"};
    if (op->ne[0] > lnship_max_row(w32 ? 3 : 1, w32 ? 0 : node_mode(op))) return {false, "lnship_row_too_long"};
    return v;
}

// common/lns-op-support.h:43-50 plus cuda/lns-cuda-ops.cpp:82-89
static verdict check_binary(const ggml_tensor *op) {
    verdict v = f32_result(op, {is_f32(op->src[0]) && is_f32(op->src[1]), "binary_requires_f32_srcs"});
    if (v.ok && !can_repeat(op->src[1], op->src[0])) return {false, "lnship_binary_requires_repeatable_src1"};
    return v;
}

// common/lns-op-support.h:142-170 (SWIGLU only)
static verdict check_swiglu(const ggml_tensor *op) {
    const ggml_tensor *a = op->src[0], *b = op->src[1];
    auto rows_dense = [](const ggml_tensor *t) {   // ggml_is_contiguous_1
        return t->nb[0] == ggml_type_size(t->type) && (t->ne[2] == 1 || t->nb[2] == t->nb[1] * (size_t)t->ne[1]) &&
               (t->ne[3] == 1 || t->nb[3] == t->nb[2] * (size_t)t->ne[2]);
    };
    if (!is_f32(a) || !is_f32(op)) return {false, "glu_requires_f32_src0_and_dst"};
    if (!rows_dense(a) || !rows_dense(op)) return {false, "glu_requires_contiguous_rows"};
    if (b)
        return {is_f32(b) && rows_dense(b) && b->ne[0] == a->ne[0] && nrows(b) == nrows(a) && op->ne[0] == a->ne[0] &&
                    nrows(op) == nrows(a),
                "glu_split_requires_matching_f32_contiguous_inputs"};
    return {a->ne[0] % 2 == 0 && op->ne[0] == a->ne[0] / 2 && nrows(op) == nrows(a),
            "glu_fused_requires_even_src0_and_half_width_dst"};
}

// common/lns-op-support.h:96-124 plus cuda/lns-cuda-ops.cpp:204-219
static verdict check_rope(const ggml_tensor *op) {
    if (!is_f32(op->src[0])) return {false, "rope_requires_src0_f32"};
    const int mode = op_i32(op, 2);
    if (mode != 0 && mode != 2) return {false, "rope_mode_unsupported"};   // normal or NEOX
    if (op_f32(op, 6) != 1.0f || op_f32(op, 7) != 0.0f || op_f32(op, 8) != 1.0f)
        return {false, "rope_scaling_unsupported"};
    const int n_dims = op_i32(op, 1);
    const ggml_tensor *ff = op->src[2];
    if (ff && (!is_f32(ff) || !contiguous(ff) || ff->ne[0] < n_dims / 2))
        return {false, "rope_freq_factors_require_contiguous_f32"};
    verdict v = f32_result(op, {true, "rope_normal_or_neox"});
    if (!v.ok) return v;
    const ggml_tensor *pos = op->src[1];
    if (!pos || !type_is(pos, "i32") || !contiguous(pos) || pos->ne[0] < op->src[0]->ne[2])
        return {false, "lnship_rope_requires_i32_positions"};
    if (n_dims <= 0 || n_dims % 2 != 0 || n_dims > op->src[0]->ne[0]) return {false, "lnship_rope_requires_even_n_dims"};
    return {true, "lnship_rope"};
}

// common/lns-op-support.h:79-84 plus cuda/lns-cuda-ops.cpp:100-102
static verdict check_scale(const ggml_tensor *op) {
    return f32_result(op, {is_f32(op->src[0]) && contiguous(op->src[0]) && contiguous(op),
                           "requires_contiguous_f32_src0_and_dst"});
}

// Data movement (CPY / CONT / DUP, GET_ROWS, SET_ROWS) is claimed only for a
// destination in, or headed for, the HBM buffer type: with host buffers the
// CPU backends run these nodes, as under the reference's GPU backend.  A
// view into an HBM tensor (a KV-cache write) must run here, since no other
// backend can write that memory.
static bool dst_in_hbm(const ggml_tensor *op) {
    if (!device_buffers()) return false;
    const bool allocated = op->buffer || (op->view_src && op->view_src->buffer);
    return !allocated || on_device(op);
}

// A source these ops read: F32 / F16 anywhere, any convertible type on the host.
static bool movable_src(const ggml_tensor *t) {
    return is_f32(t) || is_f16(t) || (!on_device(t) && to_f32_possible(t));
}

static verdict check_copy(const ggml_tensor *op) {
    const ggml_tensor *a = op->src[0];
    if (!dst_in_hbm(op)) return {false, "lnship_copy_requires_hbm_dst"};
    if (!movable_src(a) || !(is_f32(op) || is_f16(op))) return {false, "lnship_copy_requires_f32_or_f16"};
    if (nelements(a) != nelements(op)) return {false, "lnship_copy_requires_equal_sizes"};
    return {true, "lnship_copy"};
}

// lns_get_rows (src/lns-ops.cpp:1003-1055) with an F32 destination
static verdict check_get_rows(const ggml_tensor *op) {
    const ggml_tensor *a = op->src[0], *ids = op->src[1];
    if (!dst_in_hbm(op)) return {false, "lnship_get_rows_requires_hbm_dst"};
    if (!is_f32(op) || !movable_src(a) || !ids || !type_is(ids, "i32"))
        return {false, "get_rows_requires_f32_dst_and_convertible_src0"};
    if (a->ne[2] != ids->ne[1] || a->ne[3] != ids->ne[2] || ids->ne[3] != 1 || op->ne[0] != a->ne[0] ||
        op->ne[1] != ids->ne[0] || op->ne[2] != ids->ne[1] || op->ne[3] != ids->ne[2])
        return {false, "lnship_get_rows_shape"};
    return {true, "lnship_get_rows"};
}

// ggml's SET_ROWS: F32 rows into an F32 / F16 destination at int64 / int32 indices
static verdict check_set_rows(const ggml_tensor *op) {
    const ggml_tensor *b = op->src[0], *c = op->src[1];
    if (!dst_in_hbm(op)) return {false, "lnship_set_rows_requires_hbm_dst"};
    if (!(is_f32(op) || is_f16(op)) || !b || !is_f32(b) || !c || !(type_is(c, "i64") || type_is(c, "i32")))
        return {false, "lnship_set_rows_requires_f32_src_and_integer_indices"};
    if (b->ne[0] != op->ne[0] || b->ne[2] != op->ne[2] || b->ne[3] != op->ne[3] || b->ne[1] != c->ne[0] ||
        c->ne[1] <= 0 || c->ne[2] <= 0 || b->ne[2] % c->ne[1] != 0 || b->ne[3] % c->ne[2] != 0 || c->ne[3] != 1)
        return {false, "lnship_set_rows_shape"};
    return {true, "lnship_set_rows"};
}

static verdict check_node(const ggml_tensor *op, bool w32) {
    switch (classify(op)) {
        case kind::view: return {true, "supported_view_or_noop"};
        case kind::mul_mat: return check_mul_mat(op, w32);
        case kind::mul_mat_id: return check_mul_mat_id(op);
        case kind::rms_norm: return check_rms_norm(op, w32);
        case kind::soft_max: return check_soft_max(op, w32);
        case kind::add:
        case kind::mul: return check_binary(op);
        case kind::swiglu: return check_swiglu(op);
        case kind::rope: return check_rope(op);
        case kind::scale: return check_scale(op);
        case kind::copy: return check_copy(op);
        case kind::get_rows: return check_get_rows(op);
        case kind::set_rows: return check_set_rows(op);
        case kind::unary: return {false, "unsupported_unary_op"};
        case kind::glu: return {false, "unsupported_glu_op"};
        default: return {false, "unsupported_op"};
    }
}

// ============================================================ Monte state

namespace monte {
using get_fn = bool (*)(uint16_t *);
using set_fn = bool (*)(uint16_t);
using reserve_fn = bool (*)(uint64_t, uint16_t *);

struct cpu_lns16 {
    get_fn get = nullptr;
    set_fn set = nullptr;
    reserve_fn reserve = nullptr;
};

// The reference's LNS16 CPU backend, when this process holds one that runs
// in monte mode: then its LFSR is the one sequence every backend draws from.
static const cpu_lns16 &cpu() {
    static const cpu_lns16 c = []() {
        cpu_lns16 r;
        r.get = (get_fn)dlsym(RTLD_DEFAULT, "ggml_backend_lns16_monte_get_state");
        r.set = (set_fn)dlsym(RTLD_DEFAULT, "ggml_backend_lns16_monte_set_state");
        r.reserve = (reserve_fn)dlsym(RTLD_DEFAULT, "ggml_backend_lns16_monte_reserve");
        uint16_t probe;
        if (!r.get || !r.set || !r.reserve || !r.get(&probe)) r = cpu_lns16{};
        return r;
    }();
    return c;
}

static std::mutex mu;
static uint16_t state = 7;   // xlns16_randombits' seed (src/lns-ops.cpp:178-195)
}  // namespace monte

// ============================================================ device state

struct dev_buffer {
    void *ptr = nullptr;
    size_t bytes = 0;
    dev_buffer() = default;
    dev_buffer(const dev_buffer &) = delete;
    dev_buffer &operator=(const dev_buffer &) = delete;
    dev_buffer(dev_buffer &&o) noexcept : ptr(o.ptr), bytes(o.bytes) { o.ptr = nullptr, o.bytes = 0; }
    ~dev_buffer() { reset(); }
    void reset() {
        if (ptr) (void)hipFree(ptr);
        ptr = nullptr;
        bytes = 0;
    }
    bool try_grow(size_t n) {
        if (n <= bytes) return true;
        if (ptr) hip_ok(hipFree(ptr), "hipFree");
        ptr = nullptr;
        bytes = 0;
        if (hipMalloc(&ptr, n) != hipSuccess) {
            (void)hipGetLastError();
            ptr = nullptr;
            return false;
        }
        bytes = n;
        return true;
    }
    void *grow(size_t n) {
        if (!try_grow(std::max<size_t>(n, 256))) {
            size_t fr = 0, tot = 0;
            (void)hipMemGetInfo(&fr, &tot);
            die("out of GPU memory allocating %zu MiB of scratch (%zu MiB free); lower GGML_LNS_HIP_CACHE_MB or the "
                "batch / context size", n >> 20, fr >> 20);
        }
        return ptr;
    }
};

struct host_buffer {   // pinned staging, grow-only
    void *ptr = nullptr;
    size_t bytes = 0;
    ~host_buffer() {
        if (ptr) (void)hipHostFree(ptr);
    }
    void *grow(size_t n) {
        n = std::max<size_t>(n, 256);
        if (n > bytes) {
            if (ptr) hip_ok(hipHostFree(ptr), "hipHostFree");
            ptr = nullptr;
            hip_ok(hipHostMalloc(&ptr, n, hipHostMallocDefault), "hipHostMalloc");
            bytes = n;
        }
        return ptr;
    }
};

enum role { R_SRC0, R_SRC1, R_SRC2, R_DST, R_LNS, R_AUX, R_COUNT };

struct weight_key {
    const void *data;
    int type;
    std::array<int64_t, GGML_MAX_DIMS> ne;
    std::array<size_t, GGML_MAX_DIMS> nb;
    explicit weight_key(const ggml_tensor *t) : data(t->data), type((int)t->type) {
        std::copy(t->ne, t->ne + GGML_MAX_DIMS, ne.begin());
        std::copy(t->nb, t->nb + GGML_MAX_DIMS, nb.begin());
    }
    bool operator<(const weight_key &o) const {
        return std::tie(data, type, ne, nb) < std::tie(o.data, o.type, o.ne, o.nb);
    }
};

struct format;

struct context {
    const format *fmt;
    int device = -1;
    hipStream_t stream = nullptr;
    std::array<dev_buffer, R_COUNT> dev;
    std::array<host_buffer, R_COUNT> host;
    std::map<weight_key, dev_buffer> weights;
    size_t budget = 0, cached = 0;
    bool full_reported = false;
    bool staging_busy = false;   // an async copy may still read the pinned staging buffers
    bool index_kernels = false;  // a get_rows / set_rows read indices on the device this graph

    explicit context(const format *f) : fmt(f) {}
    ~context();
    hipStream_t get_stream();
    float *dev_f32(role r, int64_t n) { return (float *)dev[r].grow((size_t)std::max<int64_t>(n, 1) * 4); }
    // pinned staging for host-side gathers, free of in-flight copies
    void *staging(role r, size_t bytes) {
        if (staging_busy) {
            hip_ok(hipStreamSynchronize(get_stream()), "hipStreamSynchronize");
            staging_busy = false;
        }
        return host[r].grow(bytes);
    }
    const float *upload(const ggml_tensor *t, role r);
    float *out_f32(ggml_tensor *t, role r);
    const void *upload_raw(const void *host, size_t bytes, role r);
    void download(const float *src, ggml_tensor *t);
    const void *lns_matrix(const ggml_tensor *t);
    void pack(const ggml_tensor *t, void *dst);
};

// ============================================================ formats

struct format {
    const char *name;
    bool w32;
    ggml_guid guid;
    ggml_backend_reg reg;
    ggml_backend_device dev;
    ggml_backend_buffer_type buft;   // the device buffer type (HBM)
    std::string buft_name;
};

static format &fmt16();
static format &fmt32();

static const char *description(const format *f) {
    static std::string d16, d32;
    static std::once_flag o16, o32;
    std::string &d = f->w32 ? d32 : d16;
    std::call_once(f->w32 ? o32 : o16, [&]() {
        d = std::string("Logarithmic Number System on HIP (") + (f->w32 ? "xlns32" : "xlns16");
        if (!f->w32) {
            d += std::string(", sum=") + mode_name(sum_mode());
            if (sum_mode() == LNSHIP_MONTE) d += ", monte=pure16";
        }
        d += ")";
        hipDeviceProp_t p;
        if (hip_device() >= 0 && hipGetDeviceProperties(&p, hip_device()) == hipSuccess)
            d += std::string(" on ") + p.name + " (" + p.gcnArchName + ")";
    });
    return d.c_str();
}

static const char *audit_extra(const format *f) {
    static const std::string e = std::string("\"sum_mode\":\"") + mode_name(sum_mode()) + "\",";
    return f->w32 ? "" : e.c_str();
}

// ---- the device buffer type
// Tensors in HBM.  GGML_LNS_HIP_BUFFERS=device makes it each device's default
// buffer type, so ggml allocates the tensors of the nodes these backends run
// in device memory and the ops read and write them in place; unset (or
// "host") keeps the reference's CPU buffer type (common/lns-backend-
// framework.h:279-281), where every op uploads its inputs and downloads its
// output.  Transfers are synchronous; graph_compute has finished its work on
// the GPU when it returns.

struct dev_buf {
    void *base;
    size_t size;
    int device;
};

static bool is_lnship_buft(ggml_backend_buffer_type_t b) { return b == &fmt16().buft || b == &fmt32().buft; }

// the tensor's data lives in one of these buffers (views share their
// source's buffer)
static bool on_device(const ggml_tensor *t) {
    ggml_backend_buffer_t b = t->buffer ? t->buffer : (t->view_src ? t->view_src->buffer : nullptr);
    return b && is_lnship_buft(ggml_backend_buffer_get_type(b));
}

static dev_buf *dbuf(ggml_backend_buffer_t b) { return static_cast<dev_buf *>(b->context); }

static void dbuf_free(ggml_backend_buffer_t b) {
    dev_buf *c = dbuf(b);
    if (c->base) {
        (void)hipSetDevice(c->device);
        (void)hipFree(c->base);
    }
    delete c;
}
static void *dbuf_base(ggml_backend_buffer_t b) { return dbuf(b)->base; }
static void dbuf_memset(ggml_backend_buffer_t b, ggml_tensor *t, uint8_t v, size_t off, size_t n) {
    hip_ok(hipSetDevice(dbuf(b)->device), "hipSetDevice");
    hip_ok(hipMemset((char *)t->data + off, v, n), "hipMemset");
}
static void dbuf_set(ggml_backend_buffer_t b, ggml_tensor *t, const void *data, size_t off, size_t n) {
    hip_ok(hipSetDevice(dbuf(b)->device), "hipSetDevice");
    hip_ok(hipMemcpy((char *)t->data + off, data, n, hipMemcpyHostToDevice), "hipMemcpy H2D");
}
static void dbuf_get(ggml_backend_buffer_t b, const ggml_tensor *t, void *data, size_t off, size_t n) {
    hip_ok(hipSetDevice(dbuf(b)->device), "hipSetDevice");
    hip_ok(hipMemcpy(data, (const char *)t->data + off, n, hipMemcpyDeviceToHost), "hipMemcpy D2H");
}
// dst is in this buffer; src in another device buffer or in host memory
static bool dbuf_cpy(ggml_backend_buffer_t b, const ggml_tensor *src, ggml_tensor *dst) {
    if (!src->buffer) return false;
    ggml_backend_buffer_type_t st = ggml_backend_buffer_get_type(src->buffer);
    hipMemcpyKind kind;
    if (is_lnship_buft(st)) kind = hipMemcpyDeviceToDevice;
    else if (ggml_backend_buft_is_host(st)) kind = hipMemcpyHostToDevice;
    else return false;
    hip_ok(hipSetDevice(dbuf(b)->device), "hipSetDevice");
    hip_ok(hipMemcpy(dst->data, src->data, ggml_nbytes(src), kind), "hipMemcpy");
    return true;
}
static void dbuf_clear(ggml_backend_buffer_t b, uint8_t v) {
    hip_ok(hipSetDevice(dbuf(b)->device), "hipSetDevice");
    hip_ok(hipMemset(dbuf(b)->base, v, dbuf(b)->size), "hipMemset");
}

static ggml_backend_buffer_i dbuf_slots() {
    ggml_backend_buffer_i s;
    std::memset(&s, 0, sizeof s);
    s.free_buffer = dbuf_free;
    s.get_base = dbuf_base;
    s.memset_tensor = dbuf_memset;
    s.set_tensor = dbuf_set;
    s.get_tensor = dbuf_get;
    s.cpy_tensor = dbuf_cpy;
    s.clear = dbuf_clear;
    return s;
}

static const char *dbuft_name(ggml_backend_buffer_type_t t) {
    return static_cast<format *>(t->context)->buft_name.c_str();
}
static ggml_backend_buffer_t dbuft_alloc(ggml_backend_buffer_type_t t, size_t size) {
    const int dev = hip_device();
    if (dev < 0) return nullptr;
    hip_ok(hipSetDevice(dev), "hipSetDevice");
    void *p = nullptr;
    if (hipMalloc(&p, std::max<size_t>(size, 256)) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;
    }
    return ggml_backend_buffer_init(t, dbuf_slots(), new dev_buf{p, size, dev}, size);
}
static size_t dbuft_alignment(ggml_backend_buffer_type_t) { return 256; }
static bool dbuft_is_host(ggml_backend_buffer_type_t) { return false; }

static ggml_backend_buffer_type_i dbuft_slots() {
    ggml_backend_buffer_type_i s;
    std::memset(&s, 0, sizeof s);
    s.get_name = dbuft_name;
    s.alloc_buffer = dbuft_alloc;
    s.get_alignment = dbuft_alignment;
    s.is_host = dbuft_is_host;
    return s;
}

static bool device_buffers() {
    static const bool on = []() {
        const char *v = std::getenv("GGML_LNS_HIP_BUFFERS");
        if (!v || !v[0] || !std::strcmp(v, "host")) return false;
        if (!std::strcmp(v, "device")) return true;
        die("GGML_LNS_HIP_BUFFERS must be host or device (got '%s')", v);
    }();
    return on;
}

// ---- backend slots

static const char *backend_name(ggml_backend_t b) { return static_cast<context *>(b->context)->fmt->name; }

static void backend_free(ggml_backend_t b) {
    delete static_cast<context *>(b->context);
    delete b;
}

static void run_node(context &ctx, ggml_tensor *node);
static int run_fused(context &ctx, ggml_cgraph *g, int i);
static bool fuse_enabled();

static ggml_status backend_graph_compute(ggml_backend_t b, ggml_cgraph *g) {
    context &ctx = *static_cast<context *>(b->context);
    for (int i = 0; i < g->n_nodes; i++) {
        ggml_tensor *node = g->nodes[i];
        if ((node->flags & GGML_TENSOR_FLAG_COMPUTE) == 0) continue;
        if (classify(node) == kind::view || nelements(node) == 0) continue;
        if (fuse_enabled()) {   // nodes i .. i + n - 1 in one launch
            if (const int n = run_fused(ctx, g, i)) {
                i += n - 1;
                continue;
            }
        }
        run_node(ctx, node);
    }
    // results in device buffers are complete before ggml reads or copies them
    if (ctx.stream) hip_ok(hipStreamSynchronize(ctx.get_stream()), "hipStreamSynchronize");
    if (ctx.index_kernels) {   // the reference asserts on a row index out of range (src/lns-ops.cpp:1024)
        ctx.index_kernels = false;
        int64_t bad = 0;
        if (lnship_index_error(&bad, ctx.get_stream()) == 1)
            die("%s: GET_ROWS / SET_ROWS row index %lld out of range", ctx.fmt->name, (long long)bad);
    }
    return GGML_STATUS_SUCCESS;
}

static ggml_backend_i backend_slots() {
    ggml_backend_i s;
    std::memset(&s, 0, sizeof s);
    s.get_name = backend_name;
    s.free = backend_free;
    s.graph_compute = backend_graph_compute;
    return s;
}

static ggml_backend_t init_backend(format *f) {
    if (hip_device() < 0) return nullptr;
    ggml_backend *b = new ggml_backend;
    b->guid = &f->guid;
    b->iface = backend_slots();
    b->device = &f->dev;
    b->context = new context(f);
    return b;
}

// ---- device slots

static format *fmt_of(ggml_backend_dev_t d) { return static_cast<format *>(d->context); }

static const char *dev_name(ggml_backend_dev_t d) { return fmt_of(d)->name; }
static const char *dev_description(ggml_backend_dev_t d) { return description(fmt_of(d)); }

static void dev_memory(ggml_backend_dev_t, size_t *free_b, size_t *total_b) {
    *free_b = *total_b = 0;
    const int dev = hip_device();
    if (dev < 0) return;
    int prev = 0;
    if (hipGetDevice(&prev) != hipSuccess) prev = dev;
    if (hipSetDevice(dev) == hipSuccess) (void)hipMemGetInfo(free_b, total_b);
    (void)hipSetDevice(prev);
}

static ggml_backend_dev_type dev_type(ggml_backend_dev_t) { return GGML_BACKEND_DEVICE_TYPE_ACCEL; }

static void dev_props(ggml_backend_dev_t d, ggml_backend_dev_props *p) {
    p->name = dev_name(d);
    p->description = dev_description(d);
    p->type = dev_type(d);
    p->device_id = nullptr;
    dev_memory(d, &p->memory_free, &p->memory_total);
    p->caps.async = false;
    p->caps.host_buffer = false;
    p->caps.buffer_from_host_ptr = true;
    p->caps.events = false;
}

static ggml_backend_t dev_init(ggml_backend_dev_t d, const char *) { return init_backend(fmt_of(d)); }
static ggml_backend_buffer_type_t dev_buft(ggml_backend_dev_t d) {
    return device_buffers() ? &fmt_of(d)->buft : ggml_backend_cpu_buffer_type();
}
static ggml_backend_buffer_t dev_from_host_ptr(ggml_backend_dev_t, void *ptr, size_t size, size_t) {
    return ggml_backend_cpu_buffer_from_ptr(ptr, size);
}

static bool dev_supports_op(ggml_backend_dev_t d, const ggml_tensor *op) {
    const format *f = fmt_of(d);
    if (!device_selected(f->name)) {
        audit(f->name, audit_extra(f), op, false, "disabled_by_env");
        return false;
    }
    const verdict v = check_node(op, f->w32);
    audit(f->name, audit_extra(f), op, v.ok, v.reason);
    return v.ok && !op_disabled(op);
}

static bool dev_supports_buft(ggml_backend_dev_t, ggml_backend_buffer_type_t buft) {
    return is_lnship_buft(buft) || ggml_backend_buft_is_host(buft);
}

static ggml_backend_device_i device_slots() {
    ggml_backend_device_i s;
    std::memset(&s, 0, sizeof s);
    s.get_name = dev_name;
    s.get_description = dev_description;
    s.get_memory = dev_memory;
    s.get_type = dev_type;
    s.get_props = dev_props;
    s.init_backend = dev_init;
    s.get_buffer_type = dev_buft;
    s.buffer_from_host_ptr = dev_from_host_ptr;
    s.supports_op = dev_supports_op;
    s.supports_buft = dev_supports_buft;
    s.offload_op = dev_supports_op;
    return s;
}

// ---- registry slots

static const char *reg_name(ggml_backend_reg_t r) { return static_cast<format *>(r->context)->name; }
static size_t reg_count(ggml_backend_reg_t) { return hip_device() >= 0 ? 1 : 0; }
// The device record exists whether or not a GPU does (ggml only asks for
// indices below get_device_count; diagnostics may ask for 0 regardless).
static ggml_backend_dev_t reg_device(ggml_backend_reg_t r, size_t i) {
    if (i != 0) die("%s: device index %zu out of range", reg_name(r), i);
    return &static_cast<format *>(r->context)->dev;
}
static void *reg_proc(ggml_backend_reg_t r, const char *name) {
    if (static_cast<format *>(r->context)->w32 || !name) return nullptr;
    if (!std::strcmp(name, "ggml_backend_lnship16_monte_get_state")) return (void *)&ggml_backend_lnship16_monte_get_state;
    if (!std::strcmp(name, "ggml_backend_lnship16_monte_set_state")) return (void *)&ggml_backend_lnship16_monte_set_state;
    if (!std::strcmp(name, "ggml_backend_lnship16_monte_reserve")) return (void *)&ggml_backend_lnship16_monte_reserve;
    return nullptr;
}

static void make_format(format &f, const char *name, bool w32, const char guid_text[17]) {
    f.name = name;
    f.w32 = w32;
    std::memcpy(f.guid, guid_text, 16);
    f.reg.api_version = GGML_BACKEND_API_VERSION;
    f.reg.iface = {reg_name, reg_count, reg_device, reg_proc};
    f.reg.context = &f;
    f.dev.iface = device_slots();
    f.dev.reg = &f.reg;
    f.dev.context = &f;
    f.buft_name = std::string(name) + "_HBM";
    f.buft.iface = dbuft_slots();
    f.buft.device = &f.dev;
    f.buft.context = &f;
}

static format &fmt16() {
    static format f;
    static std::once_flag once;
    std::call_once(once, []() {
        (void)sum_mode();   // a bad GGML_LNS16_SUM fails at registration
        (void)sum_policy();   // and so does a bad LNS16_SUM_POLICY
        make_format(f, "LNSHIP16", false, "LNSHIP16-bkend--");
    });
    return f;
}

static format &fmt32() {
    static format f;
    static std::once_flag once;
    std::call_once(once, []() { make_format(f, "LNSHIP32", true, "LNSHIP32-bkend--"); });
    return f;
}

// ============================================================ context

context::~context() {
    if (device < 0) return;
    if (!weights.empty())
        std::fprintf(stderr, "ggml-lnship: %s cached %zu weight tensors (%.1f MiB)\n", fmt->name, weights.size(),
                     (double)cached / (1 << 20));
    (void)hipSetDevice(device);
    weights.clear();
    for (dev_buffer &b : dev) b.reset();
    if (stream) (void)hipStreamDestroy(stream);
}

// Nothing touches the GPU before the first op: a device that ggml registers
// but never uses costs no HBM.
hipStream_t context::get_stream() {
    if (stream) {
        hip_ok(hipSetDevice(device), "hipSetDevice");   // ggml may call from any thread
        return stream;
    }
    device = hip_device();
    if (device < 0) die("%s used without a GPU", fmt->name);
    hip_ok(hipSetDevice(device), "hipSetDevice");
    lib_ok(lnship_init(), "lnship_init");
    hip_ok(hipStreamCreateWithFlags(&stream, hipStreamNonBlocking), "hipStreamCreateWithFlags");
    size_t fr = 0, tot = 0;
    hip_ok(hipMemGetInfo(&fr, &tot), "hipMemGetInfo");
    const size_t reserve = (size_t)1 << 30;   // scratch for activations and uncached operands
    budget = fr > reserve ? fr - reserve : 0;
    if (const char *v = std::getenv("GGML_LNS_HIP_CACHE_MB")) budget = (size_t)std::max(0ll, std::atoll(v)) << 20;
    std::fprintf(stderr, "ggml-lnship: %s on GPU %d (%s), %zu MiB free, weight cache budget %zu MiB\n", fmt->name,
                 device, description(fmt), fr >> 20, budget >> 20);
    return stream;
}

const void *context::upload_raw(const void *h, size_t bytes, role r) {
    hipStream_t s = get_stream();
    void *d = dev[r].grow(bytes);
    hip_ok(hipMemcpyAsync(d, h, bytes, hipMemcpyHostToDevice, s), "hipMemcpyAsync H2D");
    staging_busy = true;
    return d;
}

static void view_of(const ggml_tensor *t, int64_t ne[4], int64_t nb[4]) {
    for (int d = 0; d < 4; d++) {
        ne[d] = t->ne[d];
        nb[d] = (int64_t)t->nb[d];
    }
}

const float *context::upload(const ggml_tensor *t, role r) {
    const int64_t n = nelements(t);
    if (on_device(t)) {
        if (is_f32(t) && contiguous(t)) return (const float *)t->data;
        if (!is_f32(t) && !is_f16(t))
            die("%s: %s tensor '%s' in device memory cannot be read as F32", fmt->name, ggml_type_name(t->type),
                t->name);
        float *d = dev_f32(r, n);
        int64_t ne[4], nb[4];
        view_of(t, ne, nb);
        lib_ok(lnship_gather_f32(t->data, is_f16(t) ? 1 : 0, ne, nb, d, get_stream()), "lnship_gather_f32");
        return d;
    }
    if (is_f32(t) && contiguous(t)) return (const float *)upload_raw(t->data, (size_t)n * 4, r);
    float *h = (float *)staging(r, (size_t)n * 4);
    gather_f32(t, h);
    return (const float *)upload_raw(h, (size_t)n * 4, r);
}

// Where an op writes t: t's own memory when it is a contiguous F32 tensor in
// a device buffer, else scratch that download() moves into t.
float *context::out_f32(ggml_tensor *t, role r) {
    if (on_device(t) && is_f32(t) && contiguous(t)) return (float *)t->data;
    return dev_f32(r, nelements(t));
}

// A host tensor holds the result before this returns (the next node, on
// any backend, may read it); a device tensor once the graph's stream has
// finished, which graph_compute waits for.
void context::download(const float *src, ggml_tensor *t) {
    hipStream_t s = get_stream();
    const int64_t n = nelements(t);
    if (on_device(t)) {
        if (src == t->data) return;
        if (contiguous(t)) {
            hip_ok(hipMemcpyAsync(t->data, src, (size_t)n * 4, hipMemcpyDeviceToDevice, s), "hipMemcpyAsync D2D");
        } else {
            int64_t ne[4], nb[4];
            view_of(t, ne, nb);
            lib_ok(lnship_scatter_f32(src, t->data, ne, nb, s), "lnship_scatter_f32");
        }
        return;
    }
    if (contiguous(t)) {
        hip_ok(hipMemcpyAsync(t->data, src, (size_t)n * 4, hipMemcpyDeviceToHost, s), "hipMemcpyAsync D2H");
        hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
        staging_busy = false;
        return;
    }
    float *h = (float *)staging(R_DST, (size_t)n * 4);
    hip_ok(hipMemcpyAsync(h, src, (size_t)n * 4, hipMemcpyDeviceToHost, s), "hipMemcpyAsync D2H");
    hip_ok(hipStreamSynchronize(s), "hipStreamSynchronize");
    staging_busy = false;
    scatter_f32(h, t);
}

// t (ne[0] = K, ne[1] = M, ne[2] * ne[3] slices) into the k8-interleaved LNS
// layout of lnship16_pack / lnship32_pack.
void context::pack(const ggml_tensor *t, void *dst) {
    hipStream_t s = get_stream();
    const int64_t K = t->ne[0], M = t->ne[1], ns = t->ne[2] * t->ne[3], n = nelements(t);
    const void *src;
    int src_f16 = 0;
    if ((is_f32(t) || is_f16(t) || lns16_codes(t, fmt->w32)) && contiguous(t)) {
        src_f16 = is_f16(t) ? 1 : type_is(t, "lns16") ? 2 : 0;   // source type of lnship16_pack
        src = on_device(t) ? t->data : upload_raw(t->data, (size_t)n * ggml_type_size(t->type), R_SRC0);
    } else {
        src = upload(t, R_SRC0);
    }
    if (fmt->w32)
        lib_ok(lnship32_pack(src, src_f16, K, K * M, (uint32_t *)dst, K, M, ns, s), "lnship32_pack");
    else
        lib_ok(lnship16_pack(src, src_f16, K, K * M, (uint16_t *)dst, K, M, ns, s), "lnship16_pack");
}

const void *context::lns_matrix(const ggml_tensor *t) {
    get_stream();   // the cache budget is known once the device is up
    const int64_t kp = (t->ne[0] + 7) & ~(int64_t)7;
    const size_t bytes = (size_t)(kp * t->ne[1] * t->ne[2] * t->ne[3]) * (fmt->w32 ? 4 : 2);
    if (is_weight(t)) {
        const weight_key key(t);
        auto it = weights.find(key);
        if (it != weights.end()) return it->second.ptr;
        if (cached + bytes <= budget) {
            dev_buffer b;
            if (b.try_grow(std::max<size_t>(bytes, 256))) {
                pack(t, b.ptr);
                cached += bytes;
                return weights.emplace(key, std::move(b)).first->second.ptr;
            }
        }
        if (!full_reported) {
            full_reported = true;
            std::fprintf(stderr, "ggml-lnship: %s weight cache full (%zu MiB cached); further weights are converted "
                                 "on every use (raise GGML_LNS_HIP_CACHE_MB)\n", fmt->name, cached >> 20);
        }
    }
    void *d = dev[R_LNS].grow(bytes);
    pack(t, d);
    return d;
}

// ============================================================ ops

static uint16_t reserve_monte(int mode, uint64_t draws) {
    if (mode != LNSHIP_MONTE) return 0;
    uint16_t start = 0;
    if (!ggml_backend_lnship16_monte_reserve(draws, &start)) die("Monte state unavailable");
    return start;
}

static void op_mul_mat(context &ctx, ggml_tensor *dst) {
    const ggml_tensor *a = dst->src[0], *b = dst->src[1];
    const bool w32 = ctx.fmt->w32;
    const int mode = node_mode(dst);
    lnship_mul_mat_args args;
    std::memset(&args, 0, sizeof args);
    args.w = ctx.lns_matrix(a);
    args.x = ctx.upload(b, R_SRC1);
    args.dst = ctx.out_f32(dst, R_DST);
    args.K = a->ne[0];
    args.M = a->ne[1];
    args.N = b->ne[1];
    args.ne02 = a->ne[2];
    args.ne03 = a->ne[3];
    args.ne12 = b->ne[2];
    args.ne13 = b->ne[3];
    if (w32) {
        lib_ok(lnship32_mul_mat(&args, ctx.get_stream()), "lnship32_mul_mat");
    } else {
        args.monte_seed =
            reserve_monte(mode, lnship16_mul_mat_draws(mode, args.K, args.M, args.N, args.ne12, args.ne13));
        lib_ok(lnship16_mul_mat(mode, &args, ctx.get_stream()), "lnship16_mul_mat");
    }
    ctx.download(args.dst, dst);
}

static void op_rms_norm(context &ctx, ggml_tensor *dst) {
    const ggml_tensor *a = dst->src[0];
    const float *x = ctx.upload(a, R_SRC0);
    float *y = ctx.out_f32(dst, R_DST);
    const int64_t nc = a->ne[0], nr = nrows(a);
    const float eps = op_f32(dst, 0);
    if (ctx.fmt->w32) {
        lib_ok(lnship32_rms_norm(x, y, nc, nr, eps, ctx.get_stream()), "lnship32_rms_norm");
    } else {
        const int mode = node_mode(dst);
        const uint16_t seed = reserve_monte(mode, lnship16_rms_norm_draws(mode, nc, nr));
        lib_ok(lnship16_rms_norm(mode, x, y, nc, nr, eps, seed, ctx.get_stream()), "lnship16_rms_norm");
    }
    ctx.download(y, dst);
}

static void op_soft_max(context &ctx, ggml_tensor *dst) {
    const ggml_tensor *a = dst->src[0], *mask = dst->src[1];
    lnship_soft_max_args args;
    std::memset(&args, 0, sizeof args);
    args.src = ctx.upload(a, R_SRC0);
    for (int i = 0; i < 4; i++) args.src_ne[i] = a->ne[i];
    if (mask && on_device(mask)) {
        // rows cut to the src row length, gathered on the device
        int64_t ne[4], nb[4];
        view_of(mask, ne, nb);
        ne[0] = a->ne[0];
        float *cut = ctx.dev_f32(R_SRC1, ne[0] * ne[1] * ne[2] * ne[3]);
        lib_ok(lnship_gather_f32(mask->data, is_f16(mask) ? 1 : 0, ne, nb, cut, ctx.get_stream()), "lnship_gather_f32");
        args.mask = cut;
        for (int i = 0; i < 4; i++) args.mask_ne[i] = ne[i];
    } else if (mask) {
        // rows cut to the src row length, packed contiguously
        const int64_t n0 = a->ne[0], rows = nrows(mask);
        float *full = (float *)ctx.staging(R_AUX, (size_t)nelements(mask) * 4);
        gather_f32(mask, full);
        float *cut = (float *)ctx.staging(R_SRC1, (size_t)(rows * n0) * 4);
        for (int64_t r = 0; r < rows; r++) std::memcpy(cut + r * n0, full + r * mask->ne[0], (size_t)n0 * 4);
        args.mask = (const float *)ctx.upload_raw(cut, (size_t)(rows * n0) * 4, R_SRC1);
        args.mask_ne[0] = n0;
        for (int i = 1; i < 4; i++) args.mask_ne[i] = mask->ne[i];
    } else {
        for (int i = 0; i < 4; i++) args.mask_ne[i] = 1;
    }
    args.scale = op_f32(dst, 0);
    args.dst = ctx.out_f32(dst, R_DST);
    if (ctx.fmt->w32) {
        lib_ok(lnship32_soft_max(&args, ctx.get_stream()), "lnship32_soft_max");
    } else {
        const int mode = node_mode(dst);
        args.monte_seed = reserve_monte(mode, lnship16_soft_max_draws(mode, a->ne[0], nrows(a)));
        lib_ok(lnship16_soft_max(mode, &args, ctx.get_stream()), "lnship16_soft_max");
    }
    // the mask staging buffers are reused by the next op only after download
    ctx.download(args.dst, dst);
}

// b repeats every nelements(b) elements of a (flat) when b matches a's
// leading dimensions and is 1 in every later one.
static bool flat_periodic(const ggml_tensor *b, const ggml_tensor *a) {
    int d = 0;
    while (d < GGML_MAX_DIMS && b->ne[d] == a->ne[d]) d++;
    for (int i = d; i < GGML_MAX_DIMS; i++)
        if (b->ne[i] != 1) return false;
    return true;
}

template <bool MUL>
static void op_binary(context &ctx, ggml_tensor *dst) {
    const ggml_tensor *a = dst->src[0], *b = dst->src[1];
    const int64_t n = nelements(a);
    const float *xa = ctx.upload(a, R_SRC0);
    const float *xb;
    int64_t nb;
    if (flat_periodic(b, a)) {
        xb = ctx.upload(b, R_SRC1);
        nb = nelements(b);
    } else {
        // ggml's general repeat, expanded on the host
        const int64_t nbe = nelements(b);
        float *bf = (float *)ctx.staging(R_AUX, (size_t)nbe * 4);
        if (on_device(b)) {
            const float *bd = ctx.upload(b, R_AUX);   // contiguous on the device
            hip_ok(hipStreamSynchronize(ctx.get_stream()), "hipStreamSynchronize");
            hip_ok(hipMemcpy(bf, bd, (size_t)nbe * 4, hipMemcpyDeviceToHost), "hipMemcpy D2H");
        } else {
            gather_f32(b, bf);
        }
        float *h = (float *)ctx.staging(R_SRC1, (size_t)n * 4);
        int64_t i = 0;
        for (int64_t i3 = 0; i3 < a->ne[3]; i3++)
            for (int64_t i2 = 0; i2 < a->ne[2]; i2++)
                for (int64_t i1 = 0; i1 < a->ne[1]; i1++)
                    for (int64_t i0 = 0; i0 < a->ne[0]; i0++)
                        h[i++] = bf[(((i3 % b->ne[3]) * b->ne[2] + i2 % b->ne[2]) * b->ne[1] + i1 % b->ne[1]) *
                                        b->ne[0] +
                                    i0 % b->ne[0]];
        xb = (const float *)ctx.upload_raw(h, (size_t)n * 4, R_SRC1);
        nb = n;
    }
    float *y = ctx.out_f32(dst, R_DST);
    if (ctx.fmt->w32) {
        if (MUL) lib_ok(lnship32_mul(xa, xb, n, nb, y, ctx.get_stream()), "lnship32_mul");
        else lib_ok(lnship32_add(xa, xb, n, nb, y, ctx.get_stream()), "lnship32_add");
    } else {
        if (MUL) lib_ok(lnship16_mul(xa, xb, n, nb, y, ctx.get_stream()), "lnship16_mul");
        else lib_ok(lnship16_add(xa, xb, n, nb, y, ctx.get_stream()), "lnship16_add");
    }
    ctx.download(y, dst);
}

static void op_swiglu(context &ctx, ggml_tensor *dst) {
    const ggml_tensor *a = dst->src[0], *b = dst->src[1];
    const int64_t ncols = dst->ne[0], nr = nrows(a);
    const float *x = ctx.upload(a, R_SRC0);
    const float *gate, *up;
    int64_t gate_ld = a->ne[0], up_ld = a->ne[0];
    if (b) {
        gate = x;
        up = ctx.upload(b, R_SRC1);
        up_ld = b->ne[0];
    } else {   // both halves in each src0 row, gate first unless swapped
        const bool swapped = op_i32(dst, 1) != 0;
        gate = x + (swapped ? ncols : 0);
        up = x + (swapped ? 0 : ncols);
    }
    float *y = ctx.out_f32(dst, R_DST);
    if (ctx.fmt->w32) lib_ok(lnship32_swiglu(gate, gate_ld, up, up_ld, y, ncols, nr, ctx.get_stream()), "lnship32_swiglu");
    else lib_ok(lnship16_swiglu(gate, gate_ld, up, up_ld, y, ncols, nr, ctx.get_stream()), "lnship16_swiglu");
    ctx.download(y, dst);
}

// t's first n elements on the host (a copy when t is in a device buffer)
template <class T>
static const T *host_elems(const ggml_tensor *t, int64_t n, std::vector<T> &keep) {
    if (!on_device(t)) return (const T *)t->data;
    keep.resize((size_t)n);
    hip_ok(hipMemcpy(keep.data(), t->data, (size_t)n * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    return keep.data();
}

static void op_rope(context &ctx, ggml_tensor *dst) {
    const ggml_tensor *a = dst->src[0];
    std::vector<int32_t> pos_h;
    std::vector<float> ff_h;
    if (on_device(dst->src[1]) || (dst->src[2] && on_device(dst->src[2])))
        hip_ok(hipStreamSynchronize(ctx.get_stream()), "hipStreamSynchronize");   // produced by earlier nodes
    const int32_t *pos = host_elems<int32_t>(dst->src[1], a->ne[2], pos_h);
    const float *ff = dst->src[2] ? host_elems<float>(dst->src[2], op_i32(dst, 1) / 2, ff_h) : nullptr;
    const int n_dims = op_i32(dst, 1), mode = op_i32(dst, 2);
    const int64_t half = n_dims / 2, ntok = a->ne[2] * a->ne[3];
    // (cos, sin) per token and pair in lns_rope's float sequence
    // (src/lns-ops.cpp:1225-1247): t = pos; theta = t / ff[p]; t *= scale
    const float theta_scale = powf(op_f32(dst, 5), -2.0f / (float)n_dims);
    std::vector<float> cs((size_t)(a->ne[2] * half * 2));
    for (int64_t i2 = 0; i2 < a->ne[2]; i2++) {
        float t = (float)pos[i2];
        for (int64_t p = 0; p < half; p++) {
            const float theta = ff ? t / ff[p] : t;
            cs[(size_t)((i2 * half + p) * 2)] = cosf(theta);
            cs[(size_t)((i2 * half + p) * 2 + 1)] = sinf(theta);
            t *= theta_scale;
        }
    }
    std::vector<int32_t> idx((size_t)ntok);
    for (int64_t i = 0; i < ntok; i++) idx[(size_t)i] = (int32_t)(i % a->ne[2]);
    const float *x = ctx.upload(a, R_SRC0);
    const float *csd = (const float *)ctx.upload_raw(cs.data(), cs.size() * 4, R_AUX);
    const int32_t *idd = (const int32_t *)ctx.upload_raw(idx.data(), idx.size() * 4, R_SRC2);
    float *y = ctx.out_f32(dst, R_DST);
    if (ctx.fmt->w32)
        lib_ok(lnship32_rope(x, a->ne[0] * a->ne[1], idd, ntok, a->ne[1], a->ne[0], n_dims, mode == 2, csd, y,
                             ctx.get_stream()),
               "lnship32_rope");
    else
        lib_ok(lnship16_rope(x, a->ne[0] * a->ne[1], idd, ntok, a->ne[1], a->ne[0], n_dims, mode == 2, csd, y,
                             ctx.get_stream()),
               "lnship16_rope");
    // cs and idx are host vectors: the copies above must finish before they go
    if (on_device(dst)) hip_ok(hipStreamSynchronize(ctx.get_stream()), "hipStreamSynchronize");
    ctx.download(y, dst);
}

static void op_scale(context &ctx, ggml_tensor *dst) {
    const ggml_tensor *a = dst->src[0];
    const float *x = ctx.upload(a, R_SRC0);
    float *y = ctx.out_f32(dst, R_DST);
    const float sc = op_f32(dst, 0), b = op_f32(dst, 1);
    if (ctx.fmt->w32) lib_ok(lnship32_scale(x, y, nelements(a), sc, b, ctx.get_stream()), "lnship32_scale");
    else lib_ok(lnship16_scale(x, y, nelements(a), sc, b, ctx.get_stream()), "lnship16_scale");
    ctx.download(y, dst);
}

// ---- data movement into HBM tensors

static void require_hbm(const context &ctx, const ggml_tensor *t) {
    if (!on_device(t)) die("%s: %s '%s' must be in the %s buffer type", ctx.fmt->name, ggml_op_desc(t), t->name,
                           ctx.fmt->buft_name.c_str());
}

static int elem_type(const ggml_tensor *t) { return is_f16(t) ? 1 : 0; }

// ne / nb of a contiguous F32 array of t's shape
static void dense_f32_view(const ggml_tensor *t, int64_t ne[4], int64_t nb[4]) {
    int64_t stride = 4;
    for (int d = 0; d < 4; d++) {
        ne[d] = t->ne[d];
        nb[d] = stride;
        stride *= t->ne[d];
    }
}

// a's elements where the device can read them: a itself when it is an F32
// or F16 tensor in HBM, else a contiguous F32 copy (upload)
static const void *device_elems(context &ctx, const ggml_tensor *a, role r, int *type, int64_t ne[4],
                                int64_t nb[4]) {
    if (on_device(a)) {
        *type = elem_type(a);
        view_of(a, ne, nb);
        return a->data;
    }
    *type = 0;
    dense_f32_view(a, ne, nb);
    return ctx.upload(a, r);
}

static void op_copy(context &ctx, ggml_tensor *dst) {
    require_hbm(ctx, dst);
    int st;
    int64_t ne[4], nb[4], dne[4], dnb[4];
    const void *x = device_elems(ctx, dst->src[0], R_SRC0, &st, ne, nb);
    view_of(dst, dne, dnb);
    lib_ok(lnship_copy(x, st, ne, nb, dst->data, elem_type(dst), dne, dnb, ctx.get_stream()), "lnship_copy");
}

// The indices of a GET_ROWS / SET_ROWS on the device, with their strides.
// Host indices are range-checked here (the reference's assert) and staged
// as a dense copy; device indices are checked by the kernel.
template <class T>
static const void *device_ids(context &ctx, const ggml_tensor *ids, int64_t limit, int64_t ne[3], int64_t nb[3]) {
    if (on_device(ids)) {
        ctx.index_kernels = true;
        for (int d = 0; d < 3; d++) {
            ne[d] = ids->ne[d];
            nb[d] = (int64_t)ids->nb[d];
        }
        return ids->data;
    }
    const int64_t n = ids->ne[0] * ids->ne[1] * ids->ne[2];
    T *h = (T *)ctx.staging(R_AUX, (size_t)std::max<int64_t>(n, 1) * sizeof(T));
    int64_t i = 0;
    for (int64_t i2 = 0; i2 < ids->ne[2]; i2++)
        for (int64_t i1 = 0; i1 < ids->ne[1]; i1++)
            for (int64_t i0 = 0; i0 < ids->ne[0]; i0++, i++) {
                std::memcpy(&h[i], (const char *)ids->data + i0 * ids->nb[0] + i1 * ids->nb[1] + i2 * ids->nb[2],
                            sizeof(T));
                if ((int64_t)h[i] < 0 || (int64_t)h[i] >= limit)
                    die("%s: row index %lld out of range [0, %lld) in '%s'", ctx.fmt->name, (long long)h[i],
                        (long long)limit, ids->name);
            }
    int64_t stride = sizeof(T);
    for (int d = 0; d < 3; d++) {
        ne[d] = ids->ne[d];
        nb[d] = stride;
        stride *= ids->ne[d];
    }
    return ctx.upload_raw(h, (size_t)std::max<int64_t>(n, 1) * sizeof(T), R_AUX);
}

// one row of t as F32 (ggml's to_float for every non-F32 type)
static void row_f32(const ggml_tensor *t, const char *row, float *out) {
    const ggml_type_traits *tr = is_f32(t) ? nullptr : ggml_get_type_traits(t->type);
    const int64_t ne0 = t->ne[0];
    if (t->nb[0] == ggml_type_size(t->type) || (tr && tr->is_quantized)) {
        if (!tr) std::memcpy(out, row, (size_t)ne0 * sizeof(float));
        else tr->to_float(row, out, ne0);
        return;
    }
    for (int64_t i = 0; i < ne0; i++) {
        if (!tr) std::memcpy(out + i, row + i * t->nb[0], sizeof(float));
        else tr->to_float(row + i * t->nb[0], out + i, 1);
    }
}

static void op_get_rows(context &ctx, ggml_tensor *dst) {
    require_hbm(ctx, dst);
    const ggml_tensor *a = dst->src[0], *ids = dst->src[1];
    int64_t dne[4], dnb[4];
    view_of(dst, dne, dnb);
    if (on_device(a)) {   // an F32 / F16 table in HBM
        int64_t ane[4], anb[4], ine[3], inb[3];
        view_of(a, ane, anb);
        const void *id = device_ids<int32_t>(ctx, ids, a->ne[1], ine, inb);
        lib_ok(lnship_get_rows(a->data, elem_type(a), ane, anb, (const int32_t *)id, ine, inb, (float *)dst->data, dnb,
                               ctx.get_stream()),
               "lnship_get_rows");
        return;
    }
    // a table in host memory (any type ggml converts): the rows are gathered
    // and converted on the host, then copied into dst
    std::vector<char> ids_h;
    const char *ib = (const char *)ids->data;
    if (on_device(ids)) {   // produced by earlier nodes
        hip_ok(hipStreamSynchronize(ctx.get_stream()), "hipStreamSynchronize");
        ids_h.resize(ggml_nbytes(ids));
        hip_ok(hipMemcpy(ids_h.data(), ids->data, ids_h.size(), hipMemcpyDeviceToHost), "hipMemcpy D2H");
        ib = ids_h.data();
    }
    const int64_t nr = ids->ne[0] * ids->ne[1] * ids->ne[2], nc = a->ne[0];
    float *h = (float *)ctx.staging(R_SRC0, (size_t)std::max<int64_t>(nr * nc, 1) * 4);
    int64_t i = 0;
    for (int64_t i12 = 0; i12 < ids->ne[2]; i12++)
        for (int64_t i11 = 0; i11 < ids->ne[1]; i11++)
            for (int64_t i10 = 0; i10 < ids->ne[0]; i10++, i++) {
                int32_t r;
                std::memcpy(&r, ib + i10 * ids->nb[0] + i11 * ids->nb[1] + i12 * ids->nb[2], 4);
                if (r < 0 || r >= a->ne[1])
                    die("%s: row index %d out of range [0, %lld) in '%s'", ctx.fmt->name, r, (long long)a->ne[1],
                        ids->name);
                row_f32(a, (const char *)a->data + r * a->nb[1] + i11 * a->nb[2] + i12 * a->nb[3], h + i * nc);
            }
    const float *x = (const float *)ctx.upload_raw(h, (size_t)std::max<int64_t>(nr * nc, 1) * 4, R_SRC0);
    ctx.download(x, dst);
}

static void op_set_rows(context &ctx, ggml_tensor *dst) {
    require_hbm(ctx, dst);
    const ggml_tensor *b = dst->src[0], *c = dst->src[1];
    int st;
    int64_t bne[4], bnb[4], ine[3], inb[3], dne[4], dnb[4];
    const void *x = device_elems(ctx, b, R_SRC0, &st, bne, bnb);   // F32 (checked)
    const bool i64 = type_is(c, "i64");
    const void *id = i64 ? device_ids<int64_t>(ctx, c, dst->ne[1], ine, inb)
                         : device_ids<int32_t>(ctx, c, dst->ne[1], ine, inb);
    view_of(dst, dne, dnb);
    lib_ok(lnship_set_rows((const float *)x, bne, bnb, id, i64 ? 1 : 0, ine, inb, dst->data, elem_type(dst), dne, dnb,
                           ctx.get_stream()),
           "lnship_set_rows");
}

// lns_mul_mat_id (src/lns-ops.cpp:394-462), lns32_mul_mat_id (src32/lns32-ops.cpp:154-215)
static void op_mul_mat_id(context &ctx, ggml_tensor *dst) {
    const ggml_tensor *a = dst->src[0], *b = dst->src[1], *ids = dst->src[2];
    lnship_mul_mat_id_args args;
    std::memset(&args, 0, sizeof args);
    args.w = ctx.lns_matrix(a);   // the experts, packed slice by slice
    args.x = ctx.upload(b, R_SRC1);
    int64_t ine[3], inb[3];
    args.ids = (const int32_t *)device_ids<int32_t>(ctx, ids, a->ne[2], ine, inb);
    args.dst = ctx.out_f32(dst, R_DST);
    args.K = a->ne[0];
    args.M = a->ne[1];
    args.n_expert = a->ne[2];
    args.n_expert_used = ids->ne[0];
    args.n_tokens = ids->ne[1];
    args.ne11 = b->ne[1];
    args.ids_ld = inb[1] / 4;
    if (ctx.fmt->w32) {
        lib_ok(lnship32_mul_mat_id(&args, ctx.get_stream()), "lnship32_mul_mat_id");
    } else {
        const int mode = node_mode(dst);
        args.monte_seed = reserve_monte(
            mode, lnship16_mul_mat_id_draws(mode, args.K, args.M, args.n_expert_used, args.n_tokens));
        lib_ok(lnship16_mul_mat_id(mode, &args, ctx.get_stream()), "lnship16_mul_mat_id");
    }
    ctx.download(args.dst, dst);
}

// ---- fused node pairs -----------------------------------------------------
// llama.cpp's graphs follow RMS_NORM with the MUL by its norm weight, and a
// MUL_MAT with the ADD of the residual.  When node i's result feeds node i + 1
// and nothing else (no other node or view reads it, and it is not a graph
// output), the pair runs as one launch (lnship16_rms_norm_mul, the mul_mat's
// residual) and node i's tensor is not written.  Each fused launch keeps the
// F32 value between the two nodes and its conversion, as the two nodes do.
// In sum32, an RMS_NORM -> MUL pair of one row whose product feeds only a
// MUL_MAT (a decode step's norm before q|k|v, up|gate or the output) runs
// with that MUL_MAT as one launch (lnship16_rms_norm_mul_mat).

// Opt-in (GGML_LNS_HIP_FUSE=1): graph_compute sees one split of a
// ggml_backend_sched graph at a time, so a reader of node i's tensor in a
// later split, on another backend, is not among the nodes scanned here.
// Callers that hand over whole graphs (or mark such tensors as outputs, as
// llama.cpp's scheduler does for tensors that cross splits) can enable it.
static bool fuse_enabled() {
    static const bool on = [] {
        const char *v = std::getenv("GGML_LNS_HIP_FUSE");
        return v && std::strcmp(v, "0") != 0 && v[0] != '\0';
    }();
    return on;
}

// the byte range a tensor's elements span
static void byte_span(const ggml_tensor *t, uintptr_t *lo, uintptr_t *hi) {
    size_t last = ggml_type_size(t->type);
    for (int d = 0; d < GGML_MAX_DIMS; d++)
        if (t->ne[d] > 1) last += (size_t)(t->ne[d] - 1) * t->nb[d];
    *lo = (uintptr_t)t->data;
    *hi = *lo + last;
}

static bool overlaps(const ggml_tensor *a, const ggml_tensor *b) {
    uintptr_t a0, a1, b0, b1;
    byte_span(a, &a0, &a1);
    byte_span(b, &b0, &b1);
    return a0 < b1 && b0 < a1;
}

static bool feeds_only(const ggml_cgraph *g, int i, const ggml_tensor *next) {
    const ggml_tensor *t = g->nodes[i];
    if (t->flags & GGML_TENSOR_FLAG_OUTPUT) return false;
    int uses = 0;
    for (int s = 0; s < GGML_MAX_SRC; s++) uses += next->src[s] == t;
    if (uses != 1) return false;
    for (int j = i + 2; j < g->n_nodes; j++) {
        const ggml_tensor *u = g->nodes[j];
        if (u->view_src == t) return false;
        for (int s = 0; s < GGML_MAX_SRC; s++)
            if (u->src[s] == t) return false;
    }
    return true;
}

// an F32 tensor (upload() gathers any layout into a dense copy)
static bool plain_f32(const ggml_tensor *t) { return t->type == GGML_TYPE_F32; }

// whether lnship16_rms_norm_mul_mat takes a row of K (sum32)
static bool rms_mul_mat_fits(int64_t K) { return K >= 1 && K <= lnship_max_row(5, LNSHIP_SUM32); }

// RMS_NORM t -> MUL next -> MUL_MAT mm of one sum32 row in one launch, when
// next feeds only mm (as its activation) and mm's output overlaps neither
// the row nor the norm weight (the kernel reads them until its last chain)
static bool run_rms_mul_mat(context &ctx, ggml_cgraph *g, int i, const ggml_tensor *w) {
    if (ctx.fmt->w32 || i + 2 >= g->n_nodes) return false;
    ggml_tensor *t = g->nodes[i], *next = g->nodes[i + 1], *mm = g->nodes[i + 2];
    if ((mm->flags & GGML_TENSOR_FLAG_COMPUTE) == 0 || classify(mm) != kind::mul_mat || mm->src[1] != next ||
        !feeds_only(g, i + 1, mm))
        return false;
    if (node_mode(t) != LNSHIP_SUM32 || node_mode(mm) != LNSHIP_SUM32 || nrows(t) != 1) return false;
    const ggml_tensor *a = mm->src[0];
    if (a->ne[0] != t->ne[0] || a->ne[2] != 1 || a->ne[3] != 1 || nelements(mm) != a->ne[1] || !plain_f32(mm))
        return false;
    // the fused kernel holds the row and h in LDS beside the tables: longer
    // rows run as the separate nodes
    if (!rms_mul_mat_fits(a->ne[0])) return false;
    if (overlaps(mm, t->src[0]) || overlaps(mm, w)) return false;
    // the weight first: packing a host weight stages it through R_SRC0
    const void *wm = ctx.lns_matrix(a);
    const float *x = ctx.upload(t->src[0], R_SRC0);
    const float *wd = ctx.upload(w, R_SRC1);
    float *y = ctx.out_f32(mm, R_DST);
    lib_ok(lnship16_rms_norm_mul_mat(LNSHIP_SUM32, x, wd, op_f32(t, 0), wm, y, a->ne[0], a->ne[1], ctx.get_stream()),
           "lnship16_rms_norm_mul_mat");
    ctx.download(y, mm);
    return true;
}

static int run_fused(context &ctx, ggml_cgraph *g, int i) {
    if (i + 1 >= g->n_nodes) return 0;
    ggml_tensor *t = g->nodes[i], *next = g->nodes[i + 1];
    if ((next->flags & GGML_TENSOR_FLAG_COMPUTE) == 0 || !feeds_only(g, i, next)) return 0;
    const kind k = classify(t), kn = classify(next);
    if (k == kind::rms_norm && kn == kind::mul && next->src[0] == t && plain_f32(t->src[0])) {
        // MUL by one weight row of ne[0] floats
        const ggml_tensor *w = next->src[1];
        if (!plain_f32(w) || w->ne[0] != t->ne[0] || nelements(w) != w->ne[0] || !same_shape(next, t)) return 0;
        if (overlaps(next, w) || (overlaps(next, t->src[0]) && next->data != t->src[0]->data)) return 0;
        if (run_rms_mul_mat(ctx, g, i, w)) return 3;
        const int64_t nc = t->ne[0], nr = nrows(t);
        const float *x = ctx.upload(t->src[0], R_SRC0);
        const float *wd = ctx.upload(w, R_SRC1);
        float *y = ctx.out_f32(next, R_DST);
        const float eps = op_f32(t, 0);
        if (ctx.fmt->w32) {
            lib_ok(lnship32_rms_norm_mul(x, wd, y, nc, nr, eps, ctx.get_stream()), "lnship32_rms_norm_mul");
        } else {
            const int mode = node_mode(t);
            const uint16_t seed = reserve_monte(mode, lnship16_rms_norm_draws(mode, nc, nr));
            lib_ok(lnship16_rms_norm_mul(mode, x, wd, y, nc, nr, eps, seed, nullptr, 0, ctx.get_stream()),
                   "lnship16_rms_norm_mul");
        }
        ctx.download(y, next);
        return 2;
    }
    if (k == kind::mul_mat && kn == kind::add) {
        // ADD of a residual of the product's shape (either operand order:
        // the xlns add is commutative)
        const ggml_tensor *r = next->src[0] == t ? next->src[1] : next->src[0];
        if (r == t || !plain_f32(r) || !same_shape(r, t) || !same_shape(next, t)) return 0;
        const ggml_tensor *a = t->src[0], *b = t->src[1];
        // the product reads b while the launch writes the sum: the output may
        // only replace the residual exactly (in place), never overlap b
        if (r == b || (b->data && overlaps(next, b))) return 0;
        if (overlaps(next, r) && (next->data != r->data || !contiguous(next) || !contiguous(r))) return 0;
        lnship_mul_mat_args args;
        std::memset(&args, 0, sizeof args);
        args.w = ctx.lns_matrix(a);
        args.x = ctx.upload(b, R_SRC1);
        args.residual = ctx.upload(r, R_AUX);
        args.dst = ctx.out_f32(next, R_DST);
        args.K = a->ne[0];
        args.M = a->ne[1];
        args.N = b->ne[1];
        args.ne02 = a->ne[2];
        args.ne03 = a->ne[3];
        args.ne12 = b->ne[2];
        args.ne13 = b->ne[3];
        if (ctx.fmt->w32) {
            lib_ok(lnship32_mul_mat(&args, ctx.get_stream()), "lnship32_mul_mat");
        } else {
            const int mode = node_mode(t);
            args.monte_seed =
                reserve_monte(mode, lnship16_mul_mat_draws(mode, args.K, args.M, args.N, args.ne12, args.ne13));
            lib_ok(lnship16_mul_mat(mode, &args, ctx.get_stream()), "lnship16_mul_mat");
        }
        ctx.download(args.dst, next);
        return 2;
    }
    return 0;
}

static void run_node(context &ctx, ggml_tensor *node) {
    switch (classify(node)) {
        case kind::mul_mat: return op_mul_mat(ctx, node);
        case kind::mul_mat_id: return op_mul_mat_id(ctx, node);
        case kind::rms_norm: return op_rms_norm(ctx, node);
        case kind::soft_max: return op_soft_max(ctx, node);
        case kind::add: return op_binary<false>(ctx, node);
        case kind::mul: return op_binary<true>(ctx, node);
        case kind::swiglu: return op_swiglu(ctx, node);
        case kind::rope: return op_rope(ctx, node);
        case kind::scale: return op_scale(ctx, node);
        case kind::copy: return op_copy(ctx, node);
        case kind::get_rows: return op_get_rows(ctx, node);
        case kind::set_rows: return op_set_rows(ctx, node);
        default: break;
    }
    die("%s: unsupported op %s (%s) in graph_compute", ctx.fmt->name, ggml_op_desc(node), node->name);
}

}  // namespace lnship_ggml

// ============================================================ exports

using namespace lnship_ggml;

extern "C" {

ggml_backend_t ggml_backend_lnship16_init(void) { return init_backend(&fmt16()); }
ggml_backend_t ggml_backend_lnship32_init(void) { return init_backend(&fmt32()); }

bool ggml_backend_is_lnship(ggml_backend_t b) {
    return b && b->guid &&
           (std::memcmp(*b->guid, fmt16().guid, 16) == 0 || std::memcmp(*b->guid, fmt32().guid, 16) == 0);
}

ggml_backend_reg_t ggml_backend_lnship16_reg(void) { return &fmt16().reg; }
ggml_backend_reg_t ggml_backend_lnship32_reg(void) { return &fmt32().reg; }

bool ggml_backend_lnship16_monte_get_state(uint16_t *state) {
    if (sum_mode() != LNSHIP_MONTE || !state) return false;
    if (monte::cpu().get) return monte::cpu().get(state);
    std::lock_guard<std::mutex> lk(monte::mu);
    *state = monte::state;
    return true;
}

bool ggml_backend_lnship16_monte_set_state(uint16_t state) {
    if (sum_mode() != LNSHIP_MONTE || state == 0) return false;
    if (monte::cpu().set) return monte::cpu().set(state);
    std::lock_guard<std::mutex> lk(monte::mu);
    monte::state = state;
    return true;
}

bool ggml_backend_lnship16_monte_reserve(uint64_t draws, uint16_t *start) {
    if (sum_mode() != LNSHIP_MONTE || !start) return false;
    if (monte::cpu().reserve) return monte::cpu().reserve(draws, start);
    std::lock_guard<std::mutex> lk(monte::mu);
    *start = monte::state;
    monte::state = lnship_lfsr_jump(monte::state, draws);
    return true;
}

bool ggml_backend_lnship16_check_op(const ggml_tensor *node, const char **reason) {
    const verdict v = check_node(node, false);
    if (reason) *reason = v.reason;
    return v.ok;
}

bool ggml_backend_lnship32_check_op(const ggml_tensor *node, const char **reason) {
    const verdict v = check_node(node, true);
    if (reason) *reason = v.reason;
    return v.ok;
}

}  // extern "C"
