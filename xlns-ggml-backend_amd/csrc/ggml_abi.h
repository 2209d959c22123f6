// The part of ggml's ABI the lnship backend touches, in one place.
//
// Pinned to ggml 90951f99af1fbebef3fbdd58ff5b8715b0bb9c43, the commit the
// reference builds against (patches/ggml-base-commit.txt:1), with the
// reference's GGML_TYPE_LNS16 patch (patches/ggml-core.patch:21-27).  ggml's
// headers are not available where this library is developed, so the layouts
// below are declared here; inside a ggml tree, build with
// -DLNSHIP_USE_GGML_HEADERS and the real headers replace every declaration,
// which makes the compiler check each field and slot this file names.
//
// Enum VALUES are the fragile part of the ABI (ggml inserts ops and types in
// the middle of its enums), so the backend never compares an op or a type
// against a number: it asks ggml for the name (ggml_op_name, ggml_op_desc,
// ggml_type_name) and matches strings.  What remains numeric here is stable
// across ggml's history: struct layouts, the vtable slot order the reference
// fills (lns-backend/common/lns-backend-framework.h:223-240, 307-323,
// 327-349), GGML_TENSOR_FLAG_COMPUTE, the device type and buffer usage enums
// and ggml_status.
#pragma once

#ifdef LNSHIP_USE_GGML_HEADERS
#include "ggml.h"
#include "ggml-backend.h"
#include "ggml-backend-impl.h"
#include "ggml-impl.h"
#else

#include <stdbool.h>
#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GGML_MAX_DIMS      4
#define GGML_MAX_OP_PARAMS 64
#define GGML_MAX_SRC       10
#define GGML_MAX_NAME      64
#define GGML_BACKEND_API_VERSION 2

// Opaque to this backend: compared only through their names.
enum ggml_type { GGML_TYPE_F32 = 0, GGML_TYPE_F16 = 1, GGML_TYPE_OPAQUE_MAX_ = 0x7fffffff };
enum ggml_op { GGML_OP_NONE = 0, GGML_OP_OPAQUE_MAX_ = 0x7fffffff };

enum ggml_status {
    GGML_STATUS_ALLOC_FAILED = -2,
    GGML_STATUS_FAILED       = -1,
    GGML_STATUS_SUCCESS      = 0,
    GGML_STATUS_ABORTED      = 1,
};

enum ggml_tensor_flag {
    GGML_TENSOR_FLAG_INPUT   = 1,
    GGML_TENSOR_FLAG_OUTPUT  = 2,
    GGML_TENSOR_FLAG_PARAM   = 4,
    GGML_TENSOR_FLAG_LOSS    = 8,
    GGML_TENSOR_FLAG_COMPUTE = 16,
};

struct ggml_backend_buffer;
typedef struct ggml_backend_buffer * ggml_backend_buffer_t;
typedef struct ggml_backend_buffer_type * ggml_backend_buffer_type_t;

struct ggml_tensor {
    enum ggml_type type;
    struct ggml_backend_buffer * buffer;
    int64_t ne[GGML_MAX_DIMS];
    size_t  nb[GGML_MAX_DIMS];
    enum ggml_op op;
    int32_t op_params[GGML_MAX_OP_PARAMS / sizeof(int32_t)];
    int32_t flags;
    struct ggml_tensor * src[GGML_MAX_SRC];
    struct ggml_tensor * view_src;
    size_t view_offs;
    void * data;
    char name[GGML_MAX_NAME];
    void * extra;
    char padding[8];
};

// Leading members of ggml-impl.h's graph; the backend reads no others.
struct ggml_cgraph {
    int size;
    int n_nodes;
    int n_leafs;
    struct ggml_tensor ** nodes;
};

typedef void (*ggml_to_float_t)(const void * x, float * y, int64_t k);
typedef void (*ggml_from_float_t)(const float * x, void * y, int64_t k);

struct ggml_type_traits {
    const char *      type_name;
    int64_t           blck_size;
    int64_t           blck_size_interleave;
    size_t            type_size;
    bool              is_quantized;
    ggml_to_float_t   to_float;
    ggml_from_float_t from_float_ref;
};

typedef uint8_t ggml_guid[16];
typedef ggml_guid * ggml_guid_t;

enum ggml_backend_buffer_usage {
    GGML_BACKEND_BUFFER_USAGE_ANY     = 0,
    GGML_BACKEND_BUFFER_USAGE_WEIGHTS = 1,
    GGML_BACKEND_BUFFER_USAGE_COMPUTE = 2,
};

enum ggml_backend_dev_type {
    GGML_BACKEND_DEVICE_TYPE_CPU,
    GGML_BACKEND_DEVICE_TYPE_GPU,
    GGML_BACKEND_DEVICE_TYPE_IGPU,
    GGML_BACKEND_DEVICE_TYPE_ACCEL,
};

struct ggml_backend_dev_caps {
    bool async;
    bool host_buffer;
    bool buffer_from_host_ptr;
    bool events;
};

struct ggml_backend_dev_props {
    const char * name;
    const char * description;
    size_t memory_free;
    size_t memory_total;
    enum ggml_backend_dev_type type;
    const char * device_id;
    struct ggml_backend_dev_caps caps;
};

typedef struct ggml_backend * ggml_backend_t;
typedef struct ggml_backend_device * ggml_backend_dev_t;
typedef struct ggml_backend_reg * ggml_backend_reg_t;
typedef struct ggml_backend_event * ggml_backend_event_t;
typedef void * ggml_backend_graph_plan_t;

// Slot order of lns-backend-framework.h:223-240 (16 slots).
struct ggml_backend_i {
    const char * (*get_name)(ggml_backend_t backend);
    void (*free)(ggml_backend_t backend);
    void (*set_tensor_async)(ggml_backend_t, struct ggml_tensor *, const void *, size_t, size_t);
    void (*get_tensor_async)(ggml_backend_t, const struct ggml_tensor *, void *, size_t, size_t);
    void (*set_tensor_2d_async)(ggml_backend_t, struct ggml_tensor *, const void *, size_t, size_t, size_t, size_t, size_t);
    void (*get_tensor_2d_async)(ggml_backend_t, const struct ggml_tensor *, void *, size_t, size_t, size_t, size_t, size_t);
    bool (*cpy_tensor_async)(ggml_backend_t, ggml_backend_t, const struct ggml_tensor *, struct ggml_tensor *);
    void (*synchronize)(ggml_backend_t);
    ggml_backend_graph_plan_t (*graph_plan_create)(ggml_backend_t, const struct ggml_cgraph *);
    void (*graph_plan_free)(ggml_backend_t, ggml_backend_graph_plan_t);
    void (*graph_plan_update)(ggml_backend_t, ggml_backend_graph_plan_t, const struct ggml_cgraph *);
    enum ggml_status (*graph_plan_compute)(ggml_backend_t, ggml_backend_graph_plan_t);
    enum ggml_status (*graph_compute)(ggml_backend_t backend, struct ggml_cgraph * cgraph);
    void (*event_record)(ggml_backend_t, ggml_backend_event_t);
    void (*event_wait)(ggml_backend_t, ggml_backend_event_t);
    void (*graph_optimize)(ggml_backend_t, struct ggml_cgraph *);
};

// lns-backend-framework.h:145-150
struct ggml_backend {
    ggml_guid_t guid;
    struct ggml_backend_i iface;
    ggml_backend_dev_t device;
    void * context;
};

// Slot order of lns-backend-framework.h:307-323 (15 slots).
struct ggml_backend_device_i {
    const char * (*get_name)(ggml_backend_dev_t dev);
    const char * (*get_description)(ggml_backend_dev_t dev);
    void (*get_memory)(ggml_backend_dev_t dev, size_t * free, size_t * total);
    enum ggml_backend_dev_type (*get_type)(ggml_backend_dev_t dev);
    void (*get_props)(ggml_backend_dev_t dev, struct ggml_backend_dev_props * props);
    ggml_backend_t (*init_backend)(ggml_backend_dev_t dev, const char * params);
    ggml_backend_buffer_type_t (*get_buffer_type)(ggml_backend_dev_t dev);
    ggml_backend_buffer_type_t (*get_host_buffer_type)(ggml_backend_dev_t dev);
    ggml_backend_buffer_t (*buffer_from_host_ptr)(ggml_backend_dev_t dev, void * ptr, size_t size, size_t max_tensor_size);
    bool (*supports_op)(ggml_backend_dev_t dev, const struct ggml_tensor * op);
    bool (*supports_buft)(ggml_backend_dev_t dev, ggml_backend_buffer_type_t buft);
    bool (*offload_op)(ggml_backend_dev_t dev, const struct ggml_tensor * op);
    ggml_backend_event_t (*event_new)(ggml_backend_dev_t dev);
    void (*event_free)(ggml_backend_dev_t dev, ggml_backend_event_t event);
    void (*event_synchronize)(ggml_backend_dev_t dev, ggml_backend_event_t event);
};

struct ggml_backend_device {
    struct ggml_backend_device_i iface;
    ggml_backend_reg_t reg;
    void * context;
};

// Slot order of lns-backend-framework.h:341-346.
struct ggml_backend_reg_i {
    const char * (*get_name)(ggml_backend_reg_t reg);
    size_t (*get_device_count)(ggml_backend_reg_t reg);
    ggml_backend_dev_t (*get_device)(ggml_backend_reg_t reg, size_t index);
    void * (*get_proc_address)(ggml_backend_reg_t reg, const char * name);
};

struct ggml_backend_reg {
    int api_version;
    struct ggml_backend_reg_i iface;
    void * context;
};

// The buffer interfaces of ggml-backend-impl.h (the device buffer type).  The
// reference's backends use ggml's CPU buffer type only, so nothing in it
// fixes these layouts; the code assigns every slot by name, which the build
// with LNSHIP_USE_GGML_HEADERS checks against ggml's own declarations.
struct ggml_backend_buffer_type_i {
    const char * (*get_name)(ggml_backend_buffer_type_t buft);
    ggml_backend_buffer_t (*alloc_buffer)(ggml_backend_buffer_type_t buft, size_t size);
    size_t (*get_alignment)(ggml_backend_buffer_type_t buft);
    size_t (*get_max_size)(ggml_backend_buffer_type_t buft);
    size_t (*get_alloc_size)(ggml_backend_buffer_type_t buft, const struct ggml_tensor * tensor);
    bool (*is_host)(ggml_backend_buffer_type_t buft);
};

struct ggml_backend_buffer_type {
    struct ggml_backend_buffer_type_i iface;
    ggml_backend_dev_t device;
    void * context;
};

struct ggml_backend_buffer_i {
    void (*free_buffer)(ggml_backend_buffer_t buffer);
    void * (*get_base)(ggml_backend_buffer_t buffer);
    enum ggml_status (*init_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor * tensor);
    void (*memset_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor * tensor, uint8_t value, size_t offset,
                          size_t size);
    void (*set_tensor)(ggml_backend_buffer_t buffer, struct ggml_tensor * tensor, const void * data, size_t offset,
                       size_t size);
    void (*get_tensor)(ggml_backend_buffer_t buffer, const struct ggml_tensor * tensor, void * data, size_t offset,
                       size_t size);
    bool (*cpy_tensor)(ggml_backend_buffer_t buffer, const struct ggml_tensor * src, struct ggml_tensor * dst);
    void (*clear)(ggml_backend_buffer_t buffer, uint8_t value);
    void (*reset)(ggml_backend_buffer_t buffer);
};

struct ggml_backend_buffer {
    struct ggml_backend_buffer_i iface;
    ggml_backend_buffer_type_t buft;
    void * context;
    size_t size;
    enum ggml_backend_buffer_usage usage;
};

// Functions the backend imports from ggml-base (resolved when the library is
// loaded into a process that has ggml).
const char * ggml_op_name(enum ggml_op op);
const char * ggml_op_desc(const struct ggml_tensor * t);
const char * ggml_type_name(enum ggml_type type);
size_t       ggml_type_size(enum ggml_type type);
int64_t      ggml_blck_size(enum ggml_type type);
const struct ggml_type_traits * ggml_get_type_traits(enum ggml_type type);
ggml_backend_buffer_type_t ggml_backend_cpu_buffer_type(void);
ggml_backend_buffer_t      ggml_backend_cpu_buffer_from_ptr(void * ptr, size_t size);
bool ggml_backend_buft_is_host(ggml_backend_buffer_type_t buft);
enum ggml_backend_buffer_usage ggml_backend_buffer_get_usage(ggml_backend_buffer_t buffer);
ggml_backend_buffer_type_t ggml_backend_buffer_get_type(ggml_backend_buffer_t buffer);
ggml_backend_buffer_t ggml_backend_buffer_init(ggml_backend_buffer_type_t buft, struct ggml_backend_buffer_i iface,
                                               void * context, size_t size);
size_t ggml_nbytes(const struct ggml_tensor * tensor);

#ifdef __cplusplus
}
#endif

#endif  // LNSHIP_USE_GGML_HEADERS
