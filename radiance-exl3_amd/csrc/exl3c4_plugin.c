/* exl3c4_plugin.c -- libexl3c4.so's radiance kernel-plugin face: the exports a radiance engine loads a kernel library
 * by (kernels/exl3r4d/rows.c:527-550), the eight EXL3 op schemas, one row per op, and the hooks that unpack the
 * engine's RadArgs into an Exl3c4Op and call exl3c4_launch. Plain C over include/exl3c4.h and include/rad_shim.h (the
 * ABI slice written from the reference's usage; its layouts are unverified, see that header).
 *
 * What has to stay as the reference has it, and is restated here in code of this file's own:
 *   - the schemas: op names, parameter specs and operand lists in order (include/exl3_abi.h:366-627) -- a loader
 *     refuses a second library whose schemas differ (include/exl3_abi.h:5-9);
 *   - the geometry rule (include/exl3_abi.h:690-755): which parameters each op requires, the dtype and codebook
 *     names, K % 128, N % 256 for gate_up and N % 128 for down, the odd class, the output widths;
 *   - moe_exl3_gate_up_down's down view: down's weight is [K, N / 2] with suh = gate_up's dn_suh
 *     (include/exl3_abi.h:751-800);
 *   - the plane extents of a table entry (include/exl3_abi.h:647-665) and the class interleave (:847-853).
 * Operand positions are not tabulated: each is found by its name in the schema (codes, codes_odd, codes_1, ...). */
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "exl3c4.h"
#include "exl3c4_dev.h"
#include "rad_shim.h"

/* the stored form of a codes table entry (exl3c4_relayout's record), as an element type of its own */
#define EXL3C4_DT_TRELLIS (RAD_DT_PRIVATE + 1)

/* ------------------------------------------------------------------ schemas */

#define PI(k, r) { (k), RAD_P_INT, (r), RAD_PROLE_NONE }
#define PS(k, r) { (k), RAD_P_STR, (r), RAD_PROLE_NONE }
#define OI(n) { (n), RAD_OPD_IN, 0 }
#define OO(n) { (n), RAD_OPD_OUT, 0 }
#define OW(n) { (n), RAD_OPD_WTAB, 0 }
#define OWO(n) { (n), RAD_OPD_WTAB, 1 }

static const RadParamSpec p_gu[] = {
    PI("M", 1), PI("N", 1), PI("K", 1), PI("n_expert", 1), PI("top_k", 1), PS("dtype", 1), PS("codebook", 1),
    PI("N_odd", 0), PI("K_odd", 0), PI("h_rot", 1), PI("a_rot", 1),
};
static const RadParamSpec p_dn[] = {
    PI("M", 1), PI("N", 1), PI("K", 1), PI("n_expert", 1), PI("top_k", 1), PS("dtype", 1), PS("codebook", 1),
    PI("N_odd", 0), PI("K_odd", 0), PI("h_rot", 1),
};
static const RadParamSpec p_pg[] = {
    PI("M", 1), PI("K", 1), PI("n_expert", 1), PI("top_k", 1), PS("dtype", 1), PI("K_odd", 0),
};
static const RadParamSpec p_gd[] = {
    PI("M", 1), PI("N", 1), PI("K", 1), PI("n_expert", 1), PI("top_k", 1), PS("dtype", 1), PS("codebook", 1),
    PI("N_odd", 0), PI("K_odd", 0),
};
#define Q4 PI("N_1", 0), PI("K_1", 0), PI("N_2", 0), PI("K_2", 0), PI("N_3", 0), PI("K_3", 0)
static const RadParamSpec p_gu4[] = {
    PI("M", 1), PI("N", 1), PI("K", 1), PI("n_expert", 1), PI("top_k", 1), PS("dtype", 1), PS("codebook", 1),
    Q4, PI("h_rot", 1), PI("a_rot", 1),
};
static const RadParamSpec p_dn4[] = {
    PI("M", 1), PI("N", 1), PI("K", 1), PI("n_expert", 1), PI("top_k", 1), PS("dtype", 1), PS("codebook", 1),
    Q4, PI("h_rot", 1),
};
static const RadParamSpec p_pg4[] = {
    PI("M", 1), PI("K", 1), PI("n_expert", 1), PI("top_k", 1), PS("dtype", 1), PI("K_1", 0), PI("K_2", 0),
    PI("K_3", 0),
};
static const RadParamSpec p_gd4[] = {
    PI("M", 1), PI("N", 1), PI("K", 1), PI("n_expert", 1), PI("top_k", 1), PS("dtype", 1), PS("codebook", 1), Q4,
};
#undef Q4

static const RadOperandSpec o_gu[] = {
    OI("a"), OW("codes"), OW("suh"), OW("suh1"), OW("svh"), OWO("dn_suh"), OI("sorted_tok"), OI("expert_offset"),
    OWO("codes_odd"), OWO("suh_odd"), OWO("suh1_odd"), OWO("svh_odd"), OWO("dn_suh_odd"), OO("h"),
};
static const RadOperandSpec o_dn[] = {
    OI("h"), OW("codes"), OW("suh"), OW("svh"), OI("sorted_tok"), OI("expert_offset"),
    OWO("codes_odd"), OWO("suh_odd"), OWO("svh_odd"), OO("y"),
};
static const RadOperandSpec o_pg[] = {
    OI("a"), OW("suh"), OW("suh1"), OI("sorted_tok"), OI("expert_offset"), OWO("suh_odd"), OWO("suh1_odd"), OO("xr"),
};
static const RadOperandSpec o_gd[] = {
    OI("a"), OW("codes"), OW("suh"), OW("suh1"), OW("svh"), OW("dn_suh"), OW("dn_codes"), OW("dn_svh"),
    OI("sorted_tok"), OI("expert_offset"),
    OWO("codes_odd"), OWO("suh_odd"), OWO("suh1_odd"), OWO("svh_odd"), OWO("dn_suh_odd"), OWO("dn_codes_odd"),
    OWO("dn_svh_odd"), OO("y"),
};
#define GU_Q(q) OW("codes_" #q), OW("suh_" #q), OW("suh1_" #q), OW("svh_" #q), OWO("dn_suh_" #q)
static const RadOperandSpec o_gu4[] = {
    OI("a"), OW("codes"), OW("suh"), OW("suh1"), OW("svh"), OWO("dn_suh"), OI("sorted_tok"), OI("expert_offset"),
    GU_Q(1), GU_Q(2), GU_Q(3), OO("h"),
};
#undef GU_Q
#define DN_Q(q) OW("codes_" #q), OW("suh_" #q), OW("svh_" #q)
static const RadOperandSpec o_dn4[] = {
    OI("h"), OW("codes"), OW("suh"), OW("svh"), OI("sorted_tok"), OI("expert_offset"), DN_Q(1), DN_Q(2), DN_Q(3),
    OO("y"),
};
#undef DN_Q
#define PG_Q(q) OW("suh_" #q), OW("suh1_" #q)
static const RadOperandSpec o_pg4[] = {
    OI("a"), OW("suh"), OW("suh1"), OI("sorted_tok"), OI("expert_offset"), PG_Q(1), PG_Q(2), PG_Q(3), OO("xr"),
    { "topk_ids", RAD_OPD_IN, 1 },
};
#undef PG_Q
#define GD_Q(q) OW("codes_" #q), OW("suh_" #q), OW("suh1_" #q), OW("svh_" #q), OW("dn_suh_" #q), \
                OW("dn_codes_" #q), OW("dn_svh_" #q)
static const RadOperandSpec o_gd4[] = {
    OI("a"), OW("codes"), OW("suh"), OW("suh1"), OW("svh"), OW("dn_suh"), OW("dn_codes"), OW("dn_svh"),
    OI("sorted_tok"), OI("expert_offset"), GD_Q(1), GD_Q(2), GD_Q(3), OO("y"),
};
#undef GD_Q

#define N_OF(a) (int)(sizeof(a) / sizeof((a)[0]))
/* schema order: 0 gate_up, 1 down, 2 prep_gu, 3 gate_up_down, then their four-class forms */
/* The schemas' doc strings are the reference's own text (include/exl3_abi.h:590-625), kept verbatim: the engine's loader
 * compares the schemas of the libraries that implement these ops and refuses a second one that declares them
 * differently (docs/OPS.md:139-150 at radiance 1.3.0), and `rad-schemas exl3ref.so <this>.so` is meant to print no
 * difference. The tests compare them with the header's text. */
static const RadOpSchema k_schema[8] = {
    { "moe_exl3_gate_up", p_gu, N_OF(p_gu), o_gu, N_OF(o_gu),
      "EXL3 routed experts, gate and up: per sorted row, a[sorted_tok/top_k] scaled by suh (suh.1 for up) "
      "and rotated, times W_hat, rotated back and scaled by svh, then f16(silu(gate) * up); with h_rot = 1 "
      "that then scaled by down's suh (dn_suh) and rotated, which is down's first step; with a_rot = 1 `a` "
      "is moe_exl3_prep_gu's xr and the input rotation is not redone. One weight table a plane a parity "
      "class, expert e at entry e/2; rows past expert_offset[n_expert] are zero. expert_w is not applied. "
      "docs/OPS-exl3.md." },
    { "moe_exl3_down", p_dn, N_OF(p_dn), o_dn, N_OF(o_dn),
      "EXL3 routed experts, down: per sorted row, h[i] scaled by suh and rotated (with h_rot = 1: h[i] as "
      "gate_up already rotated it), times W_hat, rotated back and scaled by svh, bf16. One weight table a "
      "plane a parity class, expert e at entry e/2; rows past expert_offset[n_expert] are zero. expert_w is"
      " not applied. docs/OPS-exl3.md." },
    { "moe_exl3_prep_gu", p_pg, N_OF(p_pg), o_pg, N_OF(o_pg),
      "EXL3 routed experts, gate_up's input rotation as an op: per sorted row, a[sorted_tok/top_k] scaled "
      "by suh and rotated, then by suh.1 and rotated, side by side (xr, f16 [T, 2*max(K, K_odd)]) -- what "
      "moe_exl3_gate_up with a_rot = 1 reads. Rows past expert_offset[n_expert] are zero. docs/OPS-exl3.md." },
    { "moe_exl3_gate_up_down", p_gd, N_OF(p_gd), o_gd, N_OF(o_gd),
      "EXL3 routed experts, the decode chain as one op: y = moe_exl3_down(h_rot = 1) of "
      "moe_exl3_gate_up(a_rot = 0, h_rot = 1) of a, on the same routing; dn_suh / dn_codes / dn_svh are "
      "down's planes ([K, N/2]); h and the rotated input are scratch. Rows past expert_offset[n_expert] are"
      " zero. docs/OPS-exl3.md." },
    { "moe_exl3_gate_up_mod4", p_gu4, N_OF(p_gu4), o_gu4, N_OF(o_gu4),
      "moe_exl3_gate_up over FOUR classes of experts by number mod 4 (moe_gemm_q_mod4's): class q at [N_q, "
      "K_q], expert e at entry e/4 of class e%4; otherwise moe_exl3_gate_up. docs/OPS-exl3.md." },
    { "moe_exl3_down_mod4", p_dn4, N_OF(p_dn4), o_dn4, N_OF(o_dn4),
      "moe_exl3_down over FOUR classes of experts by number mod 4 (moe_gemm_q_mod4's): class q at [N_q, "
      "K_q], expert e at entry e/4 of class e%4; otherwise moe_exl3_down. docs/OPS-exl3.md." },
    { "moe_exl3_prep_gu_mod4", p_pg4, N_OF(p_pg4), o_pg4, N_OF(o_pg4),
      "moe_exl3_prep_gu over FOUR classes of experts by number mod 4: class q's input width K_q, expert e "
      "at entry e/4 of class e%4; xr f16 [T, 2*max(K_q)]; otherwise moe_exl3_prep_gu. topk_ids (optional, "
      "i32 [M, top_k]): the router's expert of each (token, slot), the sort's input -- a speed hint only, "
      "the output does not depend on it. docs/OPS-exl3.md." },
    { "moe_exl3_gate_up_down_mod4", p_gd4, N_OF(p_gd4), o_gd4, N_OF(o_gd4),
      "moe_exl3_gate_up_down over FOUR classes of experts by number mod 4: y = moe_exl3_down_mod4(h_rot = "
      "1) of moe_exl3_gate_up_mod4(a_rot = 0, h_rot = 1) of a; class q at [N_q, K_q], expert e at entry e/4"
      " of class e%4; otherwise moe_exl3_gate_up_down. docs/OPS-exl3.md." },
};

/* schema i -> (exl3c4 op, four classes?) */
static int op_of(int i) { return i == 0 || i == 4 ? EXL3C4_GATE_UP : i == 1 || i == 5 ? EXL3C4_DOWN
                                 : i == 2 || i == 6 ? EXL3C4_PREP_GU : EXL3C4_GU_DN; }
static int mod4_of(int i) { return i >= 4; }

/* ------------------------------------------------------------------ operand positions, by name */

enum { PL_CODES, PL_SUH, PL_SUH1, PL_SVH, PL_DN_SUH, PL_DN_CODES, PL_DN_SVH, PL_N };
static const char* const k_plane[PL_N] = { "codes", "suh", "suh1", "svh", "dn_suh", "dn_codes", "dn_svh" };

static int opd_named(const RadOpSchema* s, const char* name) {
    for (int i = 0; i < s->n_operands; ++i)
        if (!strcmp(s->operands[i].name, name)) return i;
    return -1;
}
/* class c's table of plane pl: "codes" (c 0), "codes_odd" (c 1 of a two-class op), "codes_<c>" (four-class) */
static int plane_at(int si, int c, int pl) {
    char name[32];
    if (c == 0) snprintf(name, sizeof name, "%s", k_plane[pl]);
    else if (!mod4_of(si)) snprintf(name, sizeof name, "%s_odd", k_plane[pl]);
    else snprintf(name, sizeof name, "%s_%d", k_plane[pl], c);
    return c < (mod4_of(si) ? 4 : 2) ? opd_named(&k_schema[si], name) : -1;
}
static int input_at(int si) { (void)si; return 0; }             /* "a" or down's "h": always first */
static int output_at(int si) {
    const RadOpSchema* s = &k_schema[si];
    for (int i = 0; i < s->n_operands; ++i)
        if (s->operands[i].dir == RAD_OPD_OUT) return i;
    return -1;
}

/* ------------------------------------------------------------------ the geometry */

typedef struct Geom {
    int     op, mod4, n_class, bits, codebook, h_rot, a_rot;
    int64_t M, n_expert, top_k;
    int64_t rows[4], cols[4];   /* class c's weight as the op reads it (gate_up_down: gate_up's) */
    int64_t x_cols, y_cols;
} Geom;

static int bits_of(const char* dt) {
    for (int k = 2; dt && k <= 8; ++k) {
        char name[8];
        snprintf(name, sizeof name, "exl3k%d", k);
        if (!strcmp(dt, name)) return k;
    }
    return -1;
}
static int codebook_of(const char* cb) {
    if (!cb) return -1;
    if (!strcmp(cb, "mul1")) return EXL3C4_CB_MUL1;
    if (!strcmp(cb, "mcg")) return EXL3C4_CB_MCG;
    if (!strcmp(cb, "3inst")) return EXL3C4_CB_3INST;
    return -1;
}

/* Parse schema si's parameters. two: the odd class's tables are present (a two-class op's operand fact). */
static int geom(const RadParam* p, int n_p, int si, int two, Geom* g) {
    const RadOpSchema* s = &k_schema[si];
    memset(g, 0, sizeof *g);
    for (int i = 0; i < s->n_params; ++i)
        if (s->params[i].required && !rad_param_find(p, n_p, s->params[i].key)) return RAD_E_SCHEMA;
    g->op = op_of(si);
    g->mod4 = mod4_of(si);
    const int prep = g->op == EXL3C4_PREP_GU, gd = g->op == EXL3C4_GU_DN, down = g->op == EXL3C4_DOWN;
    const char* dt = rad_param_gets(p, n_p, "dtype", 0);
    const char* cb = rad_param_gets(p, n_p, "codebook", 0);
    if (!dt || (!prep && !cb)) return RAD_E_SCHEMA;
    g->bits = bits_of(dt);
    g->codebook = prep ? EXL3C4_CB_MUL1 : codebook_of(cb);
    if (g->bits < 0 || g->codebook < 0) return RAD_E_DTYPE;
    g->M = rad_param_getdim(p, n_p, "M", 0);
    g->n_expert = rad_param_geti(p, n_p, "n_expert", 0);
    g->top_k = rad_param_geti(p, n_p, "top_k", 0);
    g->h_rot = prep ? 0 : gd ? 1 : (int)rad_param_geti(p, n_p, "h_rot", -1);
    g->a_rot = g->op == EXL3C4_GATE_UP ? (int)rad_param_geti(p, n_p, "a_rot", -1) : 0;
    if ((g->h_rot != 0 && g->h_rot != 1) || (g->a_rot != 0 && g->a_rot != 1)) return RAD_E_INVAL;
    if (g->M < 1 || g->n_expert < 1 || g->top_k < 1) return RAD_E_SHAPE;
    const int64_t N = rad_param_geti(p, n_p, "N", 0), K = rad_param_geti(p, n_p, "K", 0);
    g->n_class = g->mod4 ? 4 : two ? 2 : 1;
    for (int c = 0; c < 4; ++c) {
        int64_t n = N, k = K;
        if (c > 0 && g->mod4) {
            char kn[8], kk[8];
            snprintf(kn, sizeof kn, "N_%d", c);
            snprintf(kk, sizeof kk, "K_%d", c);
            n = rad_param_geti(p, n_p, kn, N);
            k = rad_param_geti(p, n_p, kk, K);
        } else if (c == 1) {
            n = rad_param_geti(p, n_p, "N_odd", N);
            k = rad_param_geti(p, n_p, "K_odd", K);
            if (!two && (k != K || (!prep && n != N))) return RAD_E_SHAPE;   /* an odd geometry without its tables */
        }
        g->rows[c] = prep ? 0 : n;
        g->cols[c] = k;
        if (c >= g->n_class) { g->rows[c] = g->rows[0]; g->cols[c] = g->cols[0]; }
    }
    for (int c = 0; c < 4; ++c) {
        if (g->cols[c] <= 0 || g->cols[c] % 128) return RAD_E_SHAPE;
        if (!prep && (g->rows[c] <= 0 || g->rows[c] % (down ? 128 : 256))) return RAD_E_SHAPE;
        if (g->cols[c] > g->x_cols) g->x_cols = g->cols[c];
        if (g->rows[c] > g->y_cols) g->y_cols = g->rows[c];
    }
    g->y_cols = prep ? 2 * g->x_cols : gd ? g->x_cols : down ? g->y_cols : g->y_cols / 2;
    return RAD_OK;
}

/* The extents [r, c] of one table entry of plane pl for a class whose weight is [rows, cols] (dn_*: gate_up_down's
 * down planes, down's weight being [cols, rows / 2]). */
static void plane_extents(int64_t rows, int64_t cols, int pl, int64_t* r, int64_t* c) {
    switch (pl) {
    case PL_CODES:    *r = rows; *c = cols; break;
    case PL_SUH:
    case PL_SUH1:     *r = 1; *c = cols; break;
    case PL_SVH:      *r = rows; *c = 1; break;
    case PL_DN_SUH:   *r = 1; *c = rows / 2; break;
    case PL_DN_CODES: *r = cols; *c = rows / 2; break;
    default:          *r = cols; *c = 1; break;   /* PL_DN_SVH */
    }
}

/* ------------------------------------------------------------------ operands -> Exl3c4Op */

/* One plane table into (base, entry stride in bytes; 0 = the engine's pointer table). */
static int table(const RadTensor* t, int pl, int64_t entries, int64_t rows, int64_t cols, int bits, const void** base,
                 int64_t* stride) {
    int64_t er, ec, per = 1;
    plane_extents(rows, cols, pl, &er, &ec);
    if (!t || t->rank < 2 || t->shape[0] < entries) return RAD_E_SHAPE;
    for (uint32_t d = 1; d < t->rank; ++d) per *= t->shape[d];
    if (pl == PL_CODES || pl == PL_DN_CODES) {
        const int64_t bytes = exl3c4_record_bytes(er, ec, bits);
        if (bytes < 0) return RAD_E_SHAPE;
        if (t->dtype == EXL3C4_DT_TRELLIS) {          /* entries are stored records, described [rows, cols] */
            if (per != er * ec || (t->stride[0] != 0 && t->stride[0] != per)) return RAD_E_SHAPE;
            *stride = t->stride[0] != 0 ? bytes : 0;
        } else if (t->dtype == RAD_U8) {              /* a tool's stacked records, u8 [entries, bytes] */
            if (per != bytes || (t->stride[0] != 0 && t->stride[0] % 256)) return RAD_E_SHAPE;
            *stride = t->stride[0];
        } else {
            return RAD_E_DTYPE;                       /* canonical uK codes go through the layout hook first */
        }
    } else {
        if (t->dtype != RAD_F16) return RAD_E_DTYPE;
        if (per != er * ec) return RAD_E_SHAPE;
        *stride = t->stride[0] * 2;
    }
    *base = t->data;
    return RAD_OK;
}

static int build_op(const RadArgs* a, int si, Exl3c4Op* o) {
    const int op = op_of(si), mod4 = mod4_of(si);
    const RadTensor* x = rad_arg_in(a, input_at(si));
    const RadTensor* y = rad_arg_in(a, output_at(si));
    const RadTensor* srt = rad_arg_in(a, opd_named(&k_schema[si], "sorted_tok"));
    const RadTensor* off = rad_arg_in(a, opd_named(&k_schema[si], "expert_offset"));
    if (!x || !y || !srt || !off) return RAD_E_INVAL;
    /* the planes this op reads, every class's; an odd class is all there or all absent */
    int want[PL_N] = { 0 }, n_odd = 0, n_planes = 0;
    want[PL_SUH] = 1;
    if (op != EXL3C4_DOWN) want[PL_SUH1] = 1;
    if (op != EXL3C4_PREP_GU) want[PL_CODES] = want[PL_SVH] = 1;
    if (op == EXL3C4_GU_DN) want[PL_DN_SUH] = want[PL_DN_CODES] = want[PL_DN_SVH] = 1;
    for (int pl = 0; pl < PL_N; ++pl) {
        if (!want[pl]) continue;
        ++n_planes;
        for (int c = 0; c < (mod4 ? 4 : 1); ++c)
            if (!rad_arg_in(a, plane_at(si, c, pl))) return RAD_E_INVAL;
        if (!mod4) n_odd += rad_arg_in(a, plane_at(si, 1, pl)) != 0;
    }
    if (n_odd != 0 && n_odd != n_planes) return RAD_E_INVAL;
    Geom g;
    int rc = geom(a->p, a->n_p, si, n_odd != 0, &g);
    if (rc != RAD_OK) return rc;
    if (op == EXL3C4_GATE_UP && g.h_rot) {
        want[PL_DN_SUH] = 1;
        for (int c = 0; c < g.n_class; ++c)
            if (!rad_arg_in(a, plane_at(si, c, PL_DN_SUH))) return RAD_E_INVAL;
    }
    /* activations and routing */
    const int token_rows = (op == EXL3C4_GATE_UP && !g.a_rot) || op == EXL3C4_PREP_GU || op == EXL3C4_GU_DN;
    if (token_rows ? (x->dtype != RAD_F16 && x->dtype != RAD_BF16) : x->dtype != RAD_F16) return RAD_E_DTYPE;
    if (y->dtype != (op == EXL3C4_DOWN || op == EXL3C4_GU_DN ? RAD_BF16 : RAD_F16)) return RAD_E_DTYPE;
    if (srt->dtype != RAD_I32 || off->dtype != RAD_I32) return RAD_E_DTYPE;
    if (!rad_tensor_is_contiguous(srt) || !rad_tensor_is_contiguous(off)) return RAD_E_STRIDE;
    if (x->rank < 2 || y->rank < 2) return RAD_E_SHAPE;
    if (x->stride[x->rank - 1] != 1 || y->stride[y->rank - 1] != 1) return RAD_E_STRIDE;
    const int64_t T = rad_tensor_rows(y);
    if (rad_tensor_numel(srt) < T || rad_tensor_numel(off) < g.n_expert + 1) return RAD_E_SHAPE;

    memset(o, 0, sizeof *o);
    o->op = op;
    o->bits = g.bits;
    o->codebook = g.codebook;
    o->n_class = g.n_class;
    o->h_rot = g.h_rot;
    o->a_rot = g.a_rot;
    o->M = g.M;
    o->n_expert = g.n_expert;
    o->top_k = g.top_k;
    for (int c = 0; c < g.n_class; ++c) {
        Exl3c4Class* k = &o->cls[c];
        const int64_t ent = (g.n_expert - c + g.n_class - 1) / g.n_class;
        const void** base[PL_N] = { &k->codes, &k->suh, &k->suh1, &k->svh, &k->dn_suh, &o->dn[c].codes, &o->dn[c].svh };
        int64_t* st[PL_N] = { &k->codes_stride, &k->suh_stride, &k->suh1_stride, &k->svh_stride, &k->dn_suh_stride,
                              &o->dn[c].codes_stride, &o->dn[c].svh_stride };
        for (int pl = 0; pl < PL_N; ++pl) {
            if (!want[pl]) continue;
            rc = table(rad_arg_in(a, plane_at(si, c, pl)), pl, ent, g.rows[c], g.cols[c], g.bits, base[pl], st[pl]);
            if (rc != RAD_OK) return rc;
        }
        k->rows = (int32_t)g.rows[c];
        k->cols = (int32_t)g.cols[c];
        if (op == EXL3C4_GU_DN) {
            o->dn[c].rows = (int32_t)g.cols[c];
            o->dn[c].cols = (int32_t)(g.rows[c] / 2);
        }
    }
    o->x = x->data;
    o->x_dtype = x->dtype == RAD_BF16 ? EXL3C4_BF16 : EXL3C4_F16;
    o->x_rows = rad_tensor_rows(x);
    o->x_cols = rad_tensor_lastdim(x);
    o->x_pitch = rad_tensor_row_pitch(x);
    o->sorted_tok = (const int32_t*)srt->data;
    o->expert_offset = (const int32_t*)off->data;
    o->y = y->data;
    o->T = T;
    o->y_cols = rad_tensor_lastdim(y);
    o->y_pitch = rad_tensor_row_pitch(y);
    return RAD_OK;
}

/* ------------------------------------------------------------------ instance state: the counter blocks
 *
 * gate_up_down's single decode kernel orders its workgroups through a counter block that is zero when it starts and
 * that a good launch leaves zero. The gate_up_down rows' instances (RadKernelInfo::init: once per resolved instance,
 * never on the launch path) hold a pool of CTR_BLOCKS such blocks, allocated and zeroed at init, one taken per
 * (stream, output) pair on first use under a mutex: two launches that may overlap run on two streams or write two
 * outputs, so they never share a block, and two that share one are ordered on its stream (the reference's pool,
 * kernels/exl3r4d/launch.c:311-330, 464-500). A launch past the pool, or with no instance (a tool calling the hook
 * cold), runs exl3c4_launch, which zeroes counters in its scratch with one more dispatch: the same bits.
 *
 * Each block has a flag in pinned host memory that the kernel sets when one of its bounded waits gives up (the launch's
 * output is then void). The host reads it without a synchronisation: the next launch that takes the block finds it
 * set, re-zeroes the block on its stream, clears the flag and returns RAD_E_DEVICE before writing anything; the launch
 * after that runs normally. */
#define CTR_BLOCKS 16
#define FLAG_STRIDE 16                                 /* int32s between two blocks' flags (a 64-byte line each) */

typedef struct Inst {
    int32_t*        ctr;                               /* CTR_BLOCKS blocks of block_bytes, zeroed at init */
    int64_t         block_bytes;
    int32_t*        fail;                              /* pinned host flags, FLAG_STRIDE apart */
    int             used;
    RadStream       key_s[CTR_BLOCKS];
    const void*     key_o[CTR_BLOCKS];
    pthread_mutex_t mu;
} Inst;

/* Counter-block bytes of gate_up_down at a band of M tokens: the status word and a counter a sorted row, then a line a
 * token (exl3c4_ctr_bytes' layout), 256 B apart. */
static int64_t ctr_block_bytes(int64_t M, int64_t top_k) {
    return ((M * top_k + 1 + M) * EXL3C4_SYNC_STRIDE * 4 + 255) / 256 * 256;
}

static int inst_init(const RadParam* p, int n_p, int si, void** out) {
    Geom g;
    *out = NULL;
    const int two = !mod4_of(si) && (rad_param_find(p, n_p, "N_odd") || rad_param_find(p, n_p, "K_odd"));
    if (geom(p, n_p, si, two, &g) != RAD_OK) return RAD_OK;   /* the launch refuses the geometry itself */
    Inst* q = (Inst*)calloc(1, sizeof *q);
    if (!q) return RAD_OK;                             /* no instance: every launch zeroes its own counters */
    q->block_bytes = ctr_block_bytes(g.M, g.top_k);
    q->ctr = (int32_t*)exl3c4_dev_zalloc(q->block_bytes * CTR_BLOCKS);
    q->fail = (int32_t*)exl3c4_host_zalloc((int64_t)CTR_BLOCKS * FLAG_STRIDE * 4);
    if (!q->ctr || !q->fail) {
        exl3c4_dev_free(q->ctr);
        exl3c4_host_free(q->fail);
        free(q);
        return RAD_OK;
    }
    pthread_mutex_init(&q->mu, NULL);
    *out = q;
    return RAD_OK;
}

static void inst_fini(void* inst) {
    Inst* q = (Inst*)inst;
    if (!q) return;
    exl3c4_dev_free(q->ctr);
    exl3c4_host_free(q->fail);
    pthread_mutex_destroy(&q->mu);
    free(q);
}

/* This launch's block (host bookkeeping only), or -1: past the pool. */
static int block_of(Inst* q, RadStream s, const void* out) {
    int b = -1;
    pthread_mutex_lock(&q->mu);
    for (int i = 0; i < q->used && b < 0; ++i)
        if (q->key_s[i] == s && q->key_o[i] == out) b = i;
    if (b < 0 && q->used < CTR_BLOCKS) {
        b = q->used++;
        q->key_s[b] = s;
        q->key_o[b] = out;
    }
    pthread_mutex_unlock(&q->mu);
    return b;
}

int32_t exl3c4_plugin_inst_flag(void* inst, int32_t block, int32_t set) {
    Inst* q = (Inst*)inst;
    if (!q || block < 0 || block >= CTR_BLOCKS) return -1;
    volatile int32_t* f = q->fail + (int64_t)block * FLAG_STRIDE;
    const int32_t v = *f;
    if (set >= 0) *f = set;
    return v;
}

void* exl3c4_plugin_inst_block(void* inst, int32_t block, int64_t* bytes) {
    Inst* q = (Inst*)inst;
    if (bytes) *bytes = 0;
    if (!q || block < 0) return NULL;
    pthread_mutex_lock(&q->mu);
    const int n = q->used;
    pthread_mutex_unlock(&q->mu);
    if (block >= n) return NULL;
    if (bytes) *bytes = q->block_bytes;
    return q->ctr + block * (q->block_bytes / 4);
}

int32_t exl3c4_plugin_inst_blocks_used(void* inst) {
    Inst* q = (Inst*)inst;
    if (!q) return -1;
    pthread_mutex_lock(&q->mu);
    const int n = q->used;
    pthread_mutex_unlock(&q->mu);
    return n;
}

/* ------------------------------------------------------------------ hooks */

static int launch_si(const RadArgs* a, RadStream s, int si) {
    Exl3c4Op o;
    const int rc = build_op(a, si, &o);
    if (rc != RAD_OK) return rc;
    Inst* q = (Inst*)a->inst;
    if (q && o.op == EXL3C4_GU_DN && (o.T + 1 + o.M) * EXL3C4_SYNC_STRIDE * 4 <= q->block_bytes) {
        const int b = block_of(q, s, o.y);
        if (b >= 0) {
            int32_t* blk = q->ctr + b * (q->block_bytes / 4);
            volatile int32_t* f = q->fail + (int64_t)b * FLAG_STRIDE;
            if (*f) {                                  /* the block's last launch gave up a wait: its output was void */
                *f = 0;
                const int zr = exl3c4_dev_fill(blk, q->block_bytes / 4, s);
                return zr != 0 ? zr : RAD_E_DEVICE;
            }
            return exl3c4_launch_inst(&o, a->scratch, a->scratch_bytes, s, blk, q->block_bytes, (int32_t*)f);
        }
    }
    return exl3c4_launch(&o, a->scratch, a->scratch_bytes, s);
}
/* from the parameters alone, at the band top (docs/STEP0.md:142-146) */
static int64_t scratch_si(const RadArgs* a, int si) {
    Geom g;
    int two = 0;
    for (int pl = 0; !mod4_of(si) && pl < PL_N; ++pl) two |= rad_arg_in(a, plane_at(si, 1, pl)) != 0;
    two |= rad_param_find(a->p, a->n_p, "N_odd") != 0 || rad_param_find(a->p, a->n_p, "K_odd") != 0;
    const int rc = geom(a->p, a->n_p, si, two, &g);
    if (rc != RAD_OK) return rc;
    int32_t rows[4], cols[4];
    for (int c = 0; c < 4; ++c) { rows[c] = (int32_t)g.rows[c]; cols[c] = (int32_t)g.cols[c]; }
    return exl3c4_scratch_bytes_geom(g.op, g.n_class, rows, cols, g.M, g.top_k, g.n_expert);
}

/* The shape hook: every operand of a case a tool builds cold, at the band top: token or sorted rows of f16, each
 * plane table stacked [entries, r, c] in its canonical element type, the routing as valid indices, the output. */
static void desc(RadOpdDesc* d, uint32_t dt, uint32_t rank, const int64_t* shape, uint32_t fill) {
    memset(d, 0, sizeof *d);
    d->dtype = dt;
    d->rank = rank;
    for (uint32_t r = 0; r < rank; ++r) d->shape[r] = shape[r];
    d->fill = fill;
    d->idx_const = -1;
}
static int shape_si(const RadParam* p, int n_p, int si, int operand, RadOpdDesc* out) {
    Geom g;
    const RadOpSchema* s = &k_schema[si];
    const int two = !mod4_of(si) && (rad_param_find(p, n_p, "N_odd") || rad_param_find(p, n_p, "K_odd"));
    if (geom(p, n_p, si, two, &g) != RAD_OK) return RAD_E_UNSUPPORTED;
    if (operand < 0 || operand >= s->n_operands || !out) return RAD_E_SHAPE;
    const int64_t T = g.M * g.top_k;
    const char* name = s->operands[operand].name;
    if (operand == input_at(si)) {
        const int token_rows = (g.op == EXL3C4_GATE_UP && !g.a_rot) || g.op == EXL3C4_PREP_GU || g.op == EXL3C4_GU_DN;
        desc(out, RAD_F16, 2, (int64_t[]){ token_rows ? g.M : T, g.a_rot ? 2 * g.x_cols : g.x_cols }, RAD_FILL_NORMAL);
        return RAD_OK;
    }
    if (operand == output_at(si)) {
        desc(out, g.op == EXL3C4_DOWN || g.op == EXL3C4_GU_DN ? RAD_BF16 : RAD_F16, 2, (int64_t[]){ T, g.y_cols },
             RAD_FILL_NORMAL);
        return RAD_OK;
    }
    if (!strcmp(name, "sorted_tok")) {
        desc(out, RAD_I32, 1, (int64_t[]){ T }, RAD_FILL_INDEX);
        out->idx_max = T;
        return RAD_OK;
    }
    if (!strcmp(name, "expert_offset")) {
        desc(out, RAD_I32, 1, (int64_t[]){ g.n_expert + 1 }, RAD_FILL_INDEX);
        out->flags = RAD_OPD_F_IDX_CU;
        return RAD_OK;
    }
    if (!strcmp(name, "topk_ids")) {
        desc(out, RAD_I32, 2, (int64_t[]){ g.M, g.top_k }, RAD_FILL_INDEX);
        out->idx_max = g.n_expert;
        return RAD_OK;
    }
    for (int c = 0; c < 4; ++c)
        for (int pl = 0; pl < PL_N; ++pl) {
            if (plane_at(si, c, pl) != operand) continue;
            if (c >= g.n_class || (pl == PL_DN_SUH && g.op == EXL3C4_GATE_UP && !g.h_rot)) {   /* not read */
                memset(out, 0, sizeof *out);
                out->idx_const = -1;
                out->flags = RAD_OPD_F_ABSENT;
                return RAD_OK;
            }
            int64_t r, cl;
            plane_extents(g.rows[c], g.cols[c], pl, &r, &cl);
            const int64_t ext[3] = { (g.n_expert - c + g.n_class - 1) / g.n_class, r, cl };
            if (pl == PL_CODES || pl == PL_DN_CODES) {
                desc(out, (uint32_t)(RAD_U1 + g.bits - 1), 3, ext, RAD_FILL_INDEX);
                out->idx_max = (int64_t)1 << g.bits;
            } else {
                desc(out, RAD_F16, 3, ext, RAD_FILL_NORMAL);
            }
            return RAD_OK;
        }
    return RAD_E_SHAPE;
}

/* Which (class, plane) an operand is, or -1. */
static int plane_of(int si, int operand, int* cls) {
    for (int c = 0; c < 4; ++c)
        for (int pl = 0; pl < PL_N; ++pl)
            if (plane_at(si, c, pl) == operand) { *cls = c; return pl; }
    return -1;
}
/* The layout hooks: a codes entry is stored as exl3c4_relayout's record (tag "exl3c4.trellis.k<K>", 256-B aligned);
 * a scale entry as the same f16 bytes. The canonical entry arrives as one plane tensor (host memory, [r, row bytes]
 * for codes). */
static int layout_si(const RadParam* p, int n_p, int si, int operand, const RadEncoding* e, const int* sel,
                     const RadTensor* pl, int n, RadLayout* out) {
    Geom g;
    int c = 0;
    const int two = !mod4_of(si) && (rad_param_find(p, n_p, "N_odd") || rad_param_find(p, n_p, "K_odd"));
    (void)e; (void)sel;
    if (geom(p, n_p, si, two, &g) != RAD_OK) return RAD_E_UNSUPPORTED;
    const int q = plane_of(si, operand, &c);
    if (q < 0 || !out || n < 1 || !pl) return RAD_E_INVAL;
    int64_t r, cl;
    plane_extents(g.rows[c], g.cols[c], q, &r, &cl);
    memset(out, 0, sizeof *out);
    out->align = 256;
    if (q == PL_CODES || q == PL_DN_CODES) {
        snprintf(out->tag, sizeof out->tag, "exl3c4.trellis.k%d", g.bits);
        out->dtype = EXL3C4_DT_TRELLIS;
        out->bytes = exl3c4_record_bytes(r, cl, g.bits);
        return out->bytes < 0 ? RAD_E_SHAPE : RAD_OK;
    }
    snprintf(out->tag, sizeof out->tag, "exl3c4.f16.vec");
    out->dtype = RAD_F16;
    out->bytes = r * cl * 2;
    return RAD_OK;
}
static int relayout_si(const RadParam* p, int n_p, int si, int operand, const RadEncoding* e, const int* sel,
                       const RadTensor* pl, int n, void* dst, int64_t dst_bytes) {
    RadLayout L;
    int c = 0;
    int rc = layout_si(p, n_p, si, operand, e, sel, pl, n, &L);
    if (rc != RAD_OK) return rc;
    if (!dst || dst_bytes < L.bytes || !pl[0].data) return RAD_E_INVAL;
    const int q = plane_of(si, operand, &c);
    if (q == PL_CODES || q == PL_DN_CODES) {
        Geom g;
        const int two = !mod4_of(si) && (rad_param_find(p, n_p, "N_odd") || rad_param_find(p, n_p, "K_odd"));
        geom(p, n_p, si, two, &g);
        int64_t r, cl;
        plane_extents(g.rows[c], g.cols[c], q, &r, &cl);
        const int64_t row_bytes = pl[0].rank >= 2 ? pl[0].stride[pl[0].rank - 2] : (cl * g.bits + 7) / 8;
        return exl3c4_relayout(pl[0].data, row_bytes, r, cl, g.bits, dst);
    }
    memcpy(dst, pl[0].data, (size_t)L.bytes);
    return RAD_OK;
}
static int unrelayout_si(const RadParam* p, int n_p, int si, int operand, const RadEncoding* e, const int* sel,
                         const void* src, int64_t src_bytes, const RadTensor* pl, int n) {
    RadLayout L;
    int c = 0;
    int rc = layout_si(p, n_p, si, operand, e, sel, pl, n, &L);
    if (rc != RAD_OK) return rc;
    if (!src || src_bytes < L.bytes || !pl[0].data) return RAD_E_INVAL;
    const int q = plane_of(si, operand, &c);
    if (q == PL_CODES || q == PL_DN_CODES) {
        Geom g;
        const int two = !mod4_of(si) && (rad_param_find(p, n_p, "N_odd") || rad_param_find(p, n_p, "K_odd"));
        geom(p, n_p, si, two, &g);
        int64_t r, cl;
        plane_extents(g.rows[c], g.cols[c], q, &r, &cl);
        const int64_t row_bytes = pl[0].rank >= 2 ? pl[0].stride[pl[0].rank - 2] : (cl * g.bits + 7) / 8;
        return exl3c4_unrelayout(src, r, cl, g.bits, pl[0].data, row_bytes);
    }
    memcpy(pl[0].data, src, (size_t)L.bytes);
    return RAD_OK;
}

/* one set of hooks per schema */
#define HOOKS(si, nm)                                                                                                \
    static int nm##_launch(const RadArgs* a, RadStream s) { return launch_si(a, s, si); }                           \
    static int64_t nm##_scratch(const RadArgs* a) { return scratch_si(a, si); }                                     \
    static int nm##_shape(const RadParam* p, int n_p, int o, RadOpdDesc* out) { return shape_si(p, n_p, si, o, out); } \
    static int nm##_layout(const RadParam* p, int n_p, int o, const RadEncoding* e, const int* sel,                \
                           const RadTensor* pl, int n, RadLayout* out) {                                            \
        return layout_si(p, n_p, si, o, e, sel, pl, n, out);                                                         \
    }                                                                                                                \
    static int nm##_relayout(const RadParam* p, int n_p, int o, const RadEncoding* e, const int* sel,              \
                             const RadTensor* pl, int n, void* dst, int64_t b) {                                    \
        return relayout_si(p, n_p, si, o, e, sel, pl, n, dst, b);                                                    \
    }                                                                                                                \
    static int nm##_unrelayout(const RadParam* p, int n_p, int o, const RadEncoding* e, const int* sel,            \
                               const void* src, int64_t b, const RadTensor* pl, int n) {                            \
        return unrelayout_si(p, n_p, si, o, e, sel, src, b, pl, n);                                                  \
    }
HOOKS(0, gu)
HOOKS(1, dn)
HOOKS(2, pg)
HOOKS(3, gd)
HOOKS(4, gu4)
HOOKS(5, dn4)
HOOKS(6, pg4)
HOOKS(7, gd4)
#undef HOOKS
/* the gate_up_down rows' instances: a counter-block pool (rank and world are not read: one GPU's instance) */
static int gd_init(const RadParam* p, int n_p, int rank, int world, void** out) { return inst_init(p, n_p, 3, out); }
static int gd4_init(const RadParam* p, int n_p, int rank, int world, void** out) { return inst_init(p, n_p, 7, out); }

/* ------------------------------------------------------------------ rows */

#define DTYPES "exl3k2 exl3k3 exl3k4 exl3k5 exl3k6 exl3k7 exl3k8"
#define CODEBOOKS "mul1 mcg 3inst"
static const RadConstraint c_gu[] = {
    RAD_CIN("h_rot", "0 1"), RAD_CIN("a_rot", "0 1"), RAD_CIN("dtype", DTYPES), RAD_CIN("codebook", CODEBOOKS),
    RAD_CDIV("K", 128), RAD_CDIV("N", 256), RAD_CLE("n_expert", 65536),
};
static const RadConstraint c_dn[] = {   /* down's k (its input width) is staged whole in LDS: at most 1536 */
    RAD_CIN("h_rot", "0 1"), RAD_CIN("dtype", DTYPES), RAD_CIN("codebook", CODEBOOKS),
    RAD_CDIV("K", 128), RAD_CLE("K", 1536), RAD_CDIV("N", 128), RAD_CLE("n_expert", 65536),
};
static const RadConstraint c_pg[] = {
    RAD_CIN("dtype", DTYPES), RAD_CDIV("K", 128), RAD_CLE("n_expert", 65536),
};
static const RadConstraint c_gd[] = {   /* down's k is N / 2 */
    RAD_CIN("dtype", DTYPES), RAD_CIN("codebook", CODEBOOKS),
    RAD_CDIV("K", 128), RAD_CDIV("N", 256), RAD_CLE("N", 3072), RAD_CLE("n_expert", 65536),
};

#define ROW_I(nm, opname, c, what, shp, dts, ini, fin)                                                            \
    { .name = "exl3c4_" #nm, .op = (opname), .family = "moe", .computes = (what), .shape = (shp), .dtypes = (dts),     \
      .domain = RAD_DOMAIN_DEVICE, .priority = 10, .constraints = (c), .n_constraints = N_OF(c),                   \
      .init = (ini), .fini = (fin), .launch = nm##_launch, .scratch = nm##_scratch, .layout = nm##_layout,         \
      .relayout = nm##_relayout, .opd_shape = nm##_shape, .unrelayout = nm##_unrelayout }
#define ROW(nm, opname, c, what, shp, dts) ROW_I(nm, opname, c, what, shp, dts, NULL, NULL)

static const RadKernelInfo k_rows[8] = {   /* row i serves schema i */
    ROW(gu, "moe_exl3_gate_up", c_gu, "gate and up, f16 h: input rotation staged in LDS, trellis decode in registers into "
        "v_mfma_f32_16x16x32_f16, split-K partial sums, output rotation, SiLU(gate)*up", "K % 128, N % 256",
        DTYPES ", " CODEBOOKS "; a f16 or bf16; h f16"),
    ROW(dn, "moe_exl3_down", c_dn, "down, bf16 y: input staged (rotated) in LDS, trellis decode into MFMA, output rotation in the "
        "workgroup", "K % 128 and K <= 1536, N % 128", DTYPES ", " CODEBOOKS "; h f16; y bf16"),
    ROW(pg, "moe_exl3_prep_gu", c_pg, "gate_up's input rotation as an op", "K % 128", DTYPES "; a f16 or bf16; xr f16"),
    ROW_I(gd, "moe_exl3_gate_up_down", c_gd, "the decode chain as one op: from 32 sorted rows both GEMMs in one kernel (down "
          "units wait on their rows' counters, in the instance's counter block), below it gate_up's GEMM then down's; "
          "the prefill path's two expert-grouped GEMMs from 8 rows an expert", "K % 128, N % 256 and N <= 3072",
          DTYPES ", " CODEBOOKS "; a f16 or bf16; y bf16", gd_init, inst_fini),
    ROW(gu4, "moe_exl3_gate_up_mod4", c_gu, "gate and up over four classes by expert number mod 4", "K % 128, N % 256",
        DTYPES ", " CODEBOOKS "; a f16 or bf16; h f16"),
    ROW(dn4, "moe_exl3_down_mod4", c_dn, "down over four classes by expert number mod 4", "K % 128 and K <= 1536, N % 128",
        DTYPES ", " CODEBOOKS "; h f16; y bf16"),
    ROW(pg4, "moe_exl3_prep_gu_mod4", c_pg, "gate_up's input rotation over four classes", "K % 128", DTYPES "; a f16 or bf16; xr f16"),
    ROW_I(gd4, "moe_exl3_gate_up_down_mod4", c_gd, "the decode chain over four classes (one kernel from 32 sorted rows, "
          "the instance's counter block)", "K % 128, N % 256 and N <= 3072", DTYPES ", " CODEBOOKS "; a f16 or bf16; y bf16",
          gd4_init, inst_fini),
};
#undef ROW

/* ------------------------------------------------------------------ exports */

static const RadPluginInfo k_info = {
    RAD_PLUGIN_KERNEL, "exl3c4", "0.1.0",
    "EXL3 routed-expert ops (moe_exl3_gate_up, moe_exl3_down, moe_exl3_prep_gu, moe_exl3_gate_up_down and their "
    "_mod4 forms) on MI355X: trellis decode in registers feeding CDNA4 MFMAs, K 2..8, codebooks mul1, mcg, 3inst",
    "gfx950",
};

uint32_t             rad_plugin_abi_version(void) { return RAD_ABI_VERSION; }
const RadPluginInfo* rad_plugin_info(void) { return &k_info; }
int                  rad_kernel_schema_count(void) { return 8; }
const RadOpSchema*   rad_kernel_schema_at(int i) { return i >= 0 && i < 8 ? &k_schema[i] : NULL; }
int                  rad_kernel_count(void) { return 8; }
const RadKernelInfo* rad_kernel_at(int i) { return i >= 0 && i < 8 ? &k_rows[i] : NULL; }
/* A launch reads and writes its operands, its scratch slice and (gate_up_down) its instance's counter block for its
 * (stream, output) pair only, so launches the engine overlaps never share state. */
int rad_kernel_concurrent(int i) { return i >= 0 && i < 8; }
