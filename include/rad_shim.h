/* rad_shim.h -- the slice of the radiance kernel-plugin ABI (version 17) that libexl3c4.so's plugin face uses.
 *
 * radiance's own headers (rad_abi.h, rad_plugin.h, rad_types.h, rad_encoding.h) are not available to this build, so
 * this header declares what the reference plugin reads and writes through them, written from its usage:
 *   kernels/exl3r4d/rows.c:360-550      RadKernelInfo rows, RadConstraint lists, RadPluginInfo, the exports
 *   kernels/exl3r4d/launch.c:110-250    RadArgs / RadTensor reading (rad_arg_in, rad_tensor_* helpers)
 *   kernels/exl3ref/rows.c:15-120       RadOpdDesc (the shape hook), RadParam lookups
 *   include/exl3_abi.h:366-627          RadOpSchema / RadParamSpec / RadOperandSpec
 *   include/exl3_encoding.h:84-125      RadEncoding (scheme, transform, planes)
 * The NAMES and the MEANING of every field follow that usage. The struct LAYOUTS and the enumerator VALUES are this
 * build's own and are NOT verified against ABI 17: a build against the real headers replaces this file and keeps
 * radiance-exl3_amd/csrc/exl3c4_plugin.c as it is. Nothing here is used by the op entry points of exl3c4.h. */
#ifndef RAD_SHIM_H
#define RAD_SHIM_H

#include <stddef.h>
#include <stdint.h>
#include <string.h>

#ifdef __cplusplus
extern "C" {
#endif

#define RAD_ABI_VERSION 17u

/* status codes (values: tests/ref/test_exl3ref.py:44) */
enum { RAD_OK = 0, RAD_E_SHAPE = -1, RAD_E_DTYPE = -2, RAD_E_ALIGN = -3, RAD_E_STRIDE = -4, RAD_E_FORMAT = -5,
       RAD_E_SCHEMA = -9, RAD_E_INVAL = -12, RAD_E_UNSUPPORTED = -18, RAD_E_SCRATCH = -20, RAD_E_DEVICE = -21 };

/* element types (the U1..U8 codes dtypes are the canonical uK planes, include/exl3_encoding.h:51-56) */
enum { RAD_DT_INVALID = 0, RAD_F32 = 1, RAD_F16 = 2, RAD_BF16 = 3, RAD_I32 = 4, RAD_I64 = 5, RAD_U8 = 6,
       RAD_U1 = 11, RAD_U2 = 12, RAD_U3 = 13, RAD_U4 = 14, RAD_U5 = 15, RAD_U6 = 16, RAD_U7 = 17,
       RAD_DT_PRIVATE = 64 /* first value a plugin may give its own stored forms */ };

typedef void* RadStream;   /* the engine's stream: a hipStream_t */

/* ---------------------------------------------------------------- parameters */
enum { RAD_P_INT = 1, RAD_P_STR = 2, RAD_P_F64 = 3 };
typedef struct RadParam {
    const char* key;
    int         kind;      /* RAD_P_* */
    int64_t     ival;      /* RAD_P_INT: the value, or a range's low bound */
    int64_t     ihi;       /* RAD_P_INT: a range's high bound (a shape hook sizes for it), 0 when not a range */
    const char* sval;      /* RAD_P_STR */
    double      fval;      /* RAD_P_F64 */
} RadParam;

static inline const RadParam* rad_param_find(const RadParam* p, int n, const char* key) {
    for (int i = 0; p && key && i < n; ++i)
        if (p[i].key && !strcmp(p[i].key, key)) return &p[i];
    return 0;
}
static inline int64_t rad_param_geti(const RadParam* p, int n, const char* key, int64_t dflt) {
    const RadParam* q = rad_param_find(p, n, key);
    return q && q->kind == RAD_P_INT ? q->ival : dflt;
}
/* a dimension: a range's high bound when the parameter is a range */
static inline int64_t rad_param_getdim(const RadParam* p, int n, const char* key, int64_t dflt) {
    const RadParam* q = rad_param_find(p, n, key);
    if (!q || q->kind != RAD_P_INT) return dflt;
    return q->ihi > q->ival ? q->ihi : q->ival;
}
static inline const char* rad_param_gets(const RadParam* p, int n, const char* key, const char* dflt) {
    const RadParam* q = rad_param_find(p, n, key);
    return q && q->kind == RAD_P_STR ? q->sval : dflt;
}

/* ---------------------------------------------------------------- schemas */
enum { RAD_OPTIONAL = 0, RAD_REQUIRED = 1 };
enum { RAD_PROLE_NONE = 0 };
enum { RAD_OPD_IN = 1, RAD_OPD_OUT = 2, RAD_OPD_WTAB = 3 };
typedef struct RadParamSpec { const char* key; int kind; int required; int role; } RadParamSpec;
typedef struct RadOperandSpec { const char* name; int dir; int optional; } RadOperandSpec;
typedef struct RadOpSchema {
    const char*           op;
    const RadParamSpec*   params;
    int                   n_params;
    const RadOperandSpec* operands;
    int                   n_operands;
    const char*           doc;
} RadOpSchema;

/* ---------------------------------------------------------------- tensors and arguments */
#define RAD_MAX_RANK 8
typedef struct RadTensor {
    void*    data;                    /* device pointer; a weight table: the pointer array (stride[0] == 0) or the
                                       * stacked buffer */
    uint32_t dtype;
    uint32_t rank;
    int64_t  shape[RAD_MAX_RANK];
    int64_t  stride[RAD_MAX_RANK];    /* elements */
} RadTensor;

typedef struct RadArgs {
    const RadParam*  p;
    int              n_p;
    const RadTensor* t;               /* operands in schema order; an absent one has data == 0 */
    int              n_t;
    void*            scratch;         /* the launch's scratch slice (256-B aligned) */
    int64_t          scratch_bytes;
    void*            inst;            /* what the row's init hook made, or 0 */
} RadArgs;

static inline const RadTensor* rad_arg_in(const RadArgs* a, int i) {
    return a && i >= 0 && i < a->n_t && a->t[i].data ? &a->t[i] : 0;
}
static inline int64_t rad_tensor_numel(const RadTensor* t) {
    int64_t n = 1;
    for (uint32_t r = 0; r < t->rank; ++r) n *= t->shape[r];
    return n;
}
static inline int64_t rad_tensor_lastdim(const RadTensor* t) { return t->rank ? t->shape[t->rank - 1] : 0; }
static inline int64_t rad_tensor_rows(const RadTensor* t) {
    return t->rank ? rad_tensor_numel(t) / (rad_tensor_lastdim(t) ? rad_tensor_lastdim(t) : 1) : 0;
}
static inline int64_t rad_tensor_row_pitch(const RadTensor* t) { return t->rank >= 2 ? t->stride[t->rank - 2] : 0; }
static inline int rad_tensor_is_contiguous(const RadTensor* t) {
    int64_t s = 1;
    for (int r = (int)t->rank - 1; r >= 0; --r) {
        if (t->shape[r] != 1 && t->stride[r] != s) return 0;
        s *= t->shape[r];
    }
    return 1;
}
static inline int rad_ptr_aligned(const void* p, uintptr_t a) { return ((uintptr_t)p % a) == 0; }

/* ---------------------------------------------------------------- encodings and stored forms */
#define RAD_ENC_STR 64
#define RAD_ENC_MAX_PLANES 8
typedef struct RadEncPlane { char name[RAD_ENC_STR]; uint32_t dtype; int tile_r, tile_c; } RadEncPlane;
typedef struct RadEncoding {
    char        scheme[RAD_ENC_STR];      /* "exl3" */
    char        transform[RAD_ENC_STR];   /* "<codebook>/h128" */
    int         n_planes;
    RadEncPlane plane[RAD_ENC_MAX_PLANES];
} RadEncoding;
/* What a layout hook answers: the stored form of one operand's entry. */
typedef struct RadLayout {
    char     tag[RAD_ENC_STR];   /* the stored form's name */
    uint32_t dtype;
    int64_t  bytes;              /* one entry */
    int64_t  align;
} RadLayout;

/* The shape hook's description of one operand (what a tool builds cold). */
enum { RAD_FILL_NONE = 0, RAD_FILL_NORMAL = 1, RAD_FILL_INDEX = 2 };
enum { RAD_OPD_F_ABSENT = 1, RAD_OPD_F_IDX_CU = 2 };
typedef struct RadOpdDesc {
    uint32_t dtype;
    uint32_t rank;
    int64_t  shape[RAD_MAX_RANK];
    uint32_t fill;
    uint32_t flags;
    int64_t  idx_max;
    int64_t  idx_const;
} RadOpdDesc;

/* ---------------------------------------------------------------- rows and plugin identity */
enum { RAD_C_LE = 1, RAD_C_GE = 2, RAD_C_EQ = 3, RAD_C_IN = 4, RAD_C_DIV = 5 };
typedef struct RadConstraint { const char* key; int kind; int64_t v; const char* set; } RadConstraint;
#define RAD_CLE(k, x)  { (k), RAD_C_LE, (x), 0 }
#define RAD_CGE(k, x)  { (k), RAD_C_GE, (x), 0 }
#define RAD_CEQ(k, x)  { (k), RAD_C_EQ, (x), 0 }
#define RAD_CDIV(k, x) { (k), RAD_C_DIV, (x), 0 }
#define RAD_CIN(k, s)  { (k), RAD_C_IN, 0, (s) }

enum { RAD_DOMAIN_HOST = 1, RAD_DOMAIN_DEVICE = 2 };
typedef struct RadKernelInfo {
    const char*          name;
    const char*          op;
    const char*          family;
    const char*          computes;
    const char*          shape;
    const char*          dtypes;
    int                  domain;
    int                  priority;
    const RadConstraint* constraints;
    int                  n_constraints;
    int     (*init)(const RadParam* p, int n_p, int rank, int world_size, void** out);
    void    (*fini)(void* inst);
    int     (*launch)(const RadArgs* a, RadStream s);
    int64_t (*scratch)(const RadArgs* a);
    int     (*layout)(const RadParam* p, int n_p, int operand, const RadEncoding* e, const int* sel,
                      const RadTensor* planes, int n_planes, RadLayout* out);
    int     (*relayout)(const RadParam* p, int n_p, int operand, const RadEncoding* e, const int* sel,
                        const RadTensor* planes, int n_planes, void* dst, int64_t dst_bytes);
    int     (*opd_shape)(const RadParam* p, int n_p, int operand, RadOpdDesc* out);
    int     (*unrelayout)(const RadParam* p, int n_p, int operand, const RadEncoding* e, const int* sel,
                          const void* src, int64_t src_bytes, const RadTensor* planes, int n_planes);
} RadKernelInfo;

enum { RAD_PLUGIN_KERNEL = 1 };
typedef struct RadPluginInfo {
    int         kind;
    const char* name;
    const char* version;
    const char* desc;
    const char* build_target;
} RadPluginInfo;

#ifdef __cplusplus
}
#endif

#endif
