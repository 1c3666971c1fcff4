/* exl3c4_route.c -- the C-ABI entry points of the routing around the routed-expert ops (router, moe_scatter,
 * moe_gather; include/exl3c4.h): the refusals, before anything is written, then the device launch
 * (exl3c4_route.hip). The contract is include/exl3_abi.h:90-158. */
#include <stdint.h>

#include "exl3c4.h"
#include "exl3c4_dev.h"

/* the scatter's workgroup holds a counter per (wave, expert) in LDS; the router holds a token's logits in registers */
#define SCATTER_MAX_EXPERTS 1024
#define ROUTER_MAX_EXPERTS 1024
/* router_topk_scatter runs as one workgroup (a wave a token) up to this many tokens */
#define FUSED_MAX_TOKENS 16

static int router_check(const void* logits, int32_t logits_dtype, int64_t n_tok, int64_t n_expert, int64_t pitch,
                        int32_t top_k, int32_t renorm, const int32_t* expert_ids, const float* expert_w) {
    if (logits_dtype != EXL3C4_F32 && logits_dtype != EXL3C4_F16 && logits_dtype != EXL3C4_BF16)
        return EXL3C4_E_DTYPE;
    if (renorm != 0 && renorm != 1) return EXL3C4_E_INVAL;
    if (n_tok < 0 || n_expert < 1 || top_k < 1 || top_k > 64 || top_k > n_expert) return EXL3C4_E_SHAPE;
    if (n_expert > ROUTER_MAX_EXPERTS) return EXL3C4_E_UNSUPPORTED;
    if (n_tok > INT32_MAX / 64) return EXL3C4_E_SHAPE;
    if (n_tok > 0 && (!logits || !expert_ids || !expert_w)) return EXL3C4_E_INVAL;
    if (pitch < n_expert) return EXL3C4_E_STRIDE;
    const int64_t esz = logits_dtype == EXL3C4_F32 ? 4 : 2;
    if ((uintptr_t)logits % (uintptr_t)esz || (uintptr_t)expert_ids % 4 || (uintptr_t)expert_w % 4)
        return EXL3C4_E_ALIGN;
    return EXL3C4_OK;
}

static int scatter_check(const int32_t* expert_ids, int64_t n_tok, int32_t top_k, int64_t n_expert,
                         const int32_t* sorted_tok, const int32_t* expert_offset, const int32_t* expert_count,
                         const int32_t* row_of, int ids_given) {
    if (n_tok < 0 || top_k < 1 || n_expert < 1) return EXL3C4_E_SHAPE;
    if (n_expert > SCATTER_MAX_EXPERTS) return EXL3C4_E_UNSUPPORTED;
    if (n_tok > INT32_MAX / top_k) return EXL3C4_E_SHAPE;
    if (!expert_offset || (n_tok > 0 && ((ids_given && !expert_ids) || !sorted_tok))) return EXL3C4_E_INVAL;
    if ((uintptr_t)expert_ids % 4 || (uintptr_t)sorted_tok % 4 || (uintptr_t)expert_offset % 4 ||
        (uintptr_t)expert_count % 4 || (uintptr_t)row_of % 4)
        return EXL3C4_E_ALIGN;
    return EXL3C4_OK;
}

int exl3c4_router_topk(const void* logits, int32_t logits_dtype, int64_t n_tok, int64_t n_expert, int64_t pitch,
                       int32_t top_k, int32_t renorm, int32_t* expert_ids, float* expert_w, void* stream) {
    const int rc = router_check(logits, logits_dtype, n_tok, n_expert, pitch, top_k, renorm, expert_ids, expert_w);
    if (rc) return rc;
    return exl3c4_dev_router(logits, logits_dtype, n_tok, (int32_t)n_expert, pitch, top_k, renorm, expert_ids,
                             expert_w, stream);
}

int exl3c4_moe_scatter(const int32_t* expert_ids, int64_t n_tok, int32_t top_k, int64_t expert_base,
                       int64_t n_expert, int32_t* sorted_tok, int32_t* expert_offset, int32_t* expert_count,
                       int32_t* row_of, void* stream) {
    const int rc = scatter_check(expert_ids, n_tok, top_k, n_expert, sorted_tok, expert_offset, expert_count, row_of,
                                 1);
    if (rc) return rc;
    return exl3c4_dev_scatter(expert_ids, n_tok * top_k, expert_base, (int32_t)n_expert, sorted_tok, expert_offset,
                              expert_count, row_of, stream);
}

int exl3c4_router_topk_scatter(const void* logits, int32_t logits_dtype, int64_t n_tok, int64_t n_expert,
                               int64_t pitch, int32_t top_k, int32_t renorm, int32_t* expert_ids, float* expert_w,
                               int32_t* sorted_tok, int32_t* expert_offset, int32_t* expert_count, int32_t* row_of,
                               void* stream) {
    int rc = router_check(logits, logits_dtype, n_tok, n_expert, pitch, top_k, renorm, expert_ids, expert_w);
    if (rc) return rc;
    rc = scatter_check(expert_ids, n_tok, top_k, n_expert, sorted_tok, expert_offset, expert_count, row_of, 1);
    if (rc) return rc;
    if (n_tok <= FUSED_MAX_TOKENS)
        return exl3c4_dev_route_scatter(logits, logits_dtype, (int32_t)n_tok, (int32_t)n_expert, pitch, top_k, renorm,
                                        expert_ids, expert_w, sorted_tok, expert_offset, expert_count, row_of, stream);
    rc = exl3c4_dev_router(logits, logits_dtype, n_tok, (int32_t)n_expert, pitch, top_k, renorm, expert_ids, expert_w,
                           stream);
    if (rc) return rc;
    return exl3c4_dev_scatter(expert_ids, n_tok * top_k, 0, (int32_t)n_expert, sorted_tok, expert_offset,
                              expert_count, row_of, stream);
}

int exl3c4_moe_gather(const void* y, int32_t y_dtype, int64_t y_pitch, const float* expert_w, const int32_t* row_of,
                      int64_t n_tok, int32_t top_k, int64_t cols, void* out, int64_t out_pitch, void* stream) {
    if (!y || !expert_w || !row_of || !out) return EXL3C4_E_INVAL;
    if (y_dtype != EXL3C4_BF16 && y_dtype != EXL3C4_F16) return EXL3C4_E_DTYPE;
    if (n_tok < 0 || top_k < 1 || cols < 1 || cols % 8) return EXL3C4_E_SHAPE;
    if (n_tok > INT32_MAX / top_k || n_tok > 0x7FFFFFFF) return EXL3C4_E_SHAPE;
    if (y_pitch < cols || out_pitch < cols) return EXL3C4_E_STRIDE;
    if ((uintptr_t)y % 16 || (y_pitch * 2) % 16 || (uintptr_t)out % 16 || (out_pitch * 2) % 16 ||
        (uintptr_t)expert_w % 4 || (uintptr_t)row_of % 4)
        return EXL3C4_E_ALIGN;
    return exl3c4_dev_gather(y, y_dtype, y_pitch, expert_w, row_of, n_tok, top_k, cols, out, out_pitch, stream);
}
