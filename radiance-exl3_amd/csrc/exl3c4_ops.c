/* exl3c4_ops.c -- the op entry points of include/exl3c4.h: refusals, scratch carving, and the launch sequence of each
 * op on the caller's stream. Plain C over the device C-ABI (exl3c4_dev.h). Nothing here allocates, synchronises or
 * reads the environment (the reference adapter's rule, kernels/exl3r4d/launch.c:1-3).
 *
 * WHAT A LAUNCH REFUSES, before anything is written (docs/OPS-exl3.md:292-301; kernels/exl3r4d/launch.c:5-14):
 *   EXL3C4_E_INVAL    an unknown op, a required operand absent, h_rot / a_rot not 0 or 1, n_class not 1, 2 or 4,
 *                     gate_up h_rot = 1 (or gate_up_down) without a class's dn_suh table
 *   EXL3C4_E_DTYPE    K outside 2..8, an unknown codebook, an activation of a dtype the op does not read
 *   EXL3C4_E_SHAPE    extents the format cannot hold (every K % 128, gate_up N % 256, down N % 128), a
 *                     non-positive count, an output not exactly the op's width, an input narrower than it reads
 *   EXL3C4_E_STRIDE   a row pitch below its width; a table's entry stride below its entry; a pitch or a stride past
 *                     2^31 - 1 (the kernels' argument block holds them in 32 bits)
 *   EXL3C4_E_ALIGN    a sorted-row input the 16-byte activation loads cannot take; a misaligned table
 *   EXL3C4_E_SCRATCH  less scratch than exl3c4_scratch_bytes asks for
 * The routing VALUES live in device memory and are not read here (that would be a synchronisation): the kernels
 * clamp every run to [0, T), so a malformed table gives wrong rows, never a stray write (launch.c:14-15). */
#include <stdint.h>
#include <string.h>

#include "exl3c4.h"
#include "exl3c4_dev.h"

#define ALIGN_UP(x, a) (((x) + (a) - 1) / (a) * (a))

_Static_assert(sizeof(Exl3c4Launch) == EXL3C4_KERNARG_BYTES && EXL3C4_KERNARG_BYTES <= EXL3C4_KERNARG_LIMIT,
               "the op kernels' argument block must fit the engine's kernel-argument slot");

static int is_gate_up(int op) { return op == EXL3C4_GATE_UP || op == EXL3C4_PREP_GU || op == EXL3C4_GU_DN; }

static int64_t max_cols(const Exl3c4Op* o) {
    int64_t m = 0;
    for (int c = 0; c < o->n_class; ++c) m = o->cls[c].cols > m ? o->cls[c].cols : m;
    return m;
}
static int64_t max_rows(const Exl3c4Op* o) {
    int64_t m = 0;
    for (int c = 0; c < o->n_class; ++c) m = o->cls[c].rows > m ? o->cls[c].rows : m;
    return m;
}

/* Rows a decode-path chunk holds at most: the least power of two >= min(M, 16). A token's top_k experts are distinct,
 * so an expert's run in a batch of M tokens holds at most M rows, and a chunk stages no more rows than a run can have
 * (at decode, M = 8: half the LDS of 16-row chunks). A routing that repeats an expert within a token makes longer runs;
 * they are cut into more chunks, with the same bits. */
static int chunk_for(int64_t M) {
    int c = 1;
    while (c < EXL3C4_CHUNK_ROWS && c < M) c <<= 1;
    return c;
}

/* Chunks of at most ch rows the runs of T sorted rows can make over n_expert experts. */
static int64_t chunk_bound(int64_t T, int64_t n_expert, int ch) {
    return T / ch + (n_expert < T ? n_expert : T) + 1;
}

/* gate_up's split-K on the decode path, from T, M and the geometry (never the routing): the most splits -- a power of
 * two, at most 16 and at most one a 128-block of k -- that keep the launch's gate_up units (chunks x n_grp x S) at
 * most GU_UNITS. A split shortens a unit's chain of code loads (and so the wait of the row's down units for its last
 * gate_up unit) and adds a unit's fixed start-up; on configs[2] (80 chunks x 8 groups) S = 4, 2560 units against
 * about 1790 resident workgroups, measured 1.7 us a layer step faster than S = 2 (every unit resident at once) and
 * 5 us faster than S = 8. Then more splits while a split's staged rows would take more LDS than GU_LDS_BUDGET (which
 * keeps 7 workgroups a CU). */
#ifndef GU_UNITS
#define GU_UNITS 4096
#endif
#ifndef GU_LDS_BUDGET
#define GU_LDS_BUDGET (20 * 1024)
#endif
static int ksplit_for(int64_t chunks, int64_t n_grp, int64_t nb_min, int64_t nb_max, int ch) {
    int s = 1;
    while (s < 16 && 2 * s <= nb_min && chunks * n_grp * 2 * s <= GU_UNITS) s *= 2;
    while (s < 16 && 2 * s <= nb_max && (int64_t)ch * (((nb_max + s - 1) / s) * 128 + 8) * 2 > GU_LDS_BUDGET) s *= 2;
    return s;
}

static int log2i(int v) {
    int l = 0;
    while ((1 << l) < v) ++l;
    return l;
}

/* The prefill path (the rotation with the chunk plan, then one GEMM kernel a projection over chunks of up to 112 rows
 * of one expert) serves a launch of at least 64 sorted rows that average at least 7/8 of a row an expert: T >= 64 and
 * 8 T >= 7 n_expert (exl3c4_prefill_min_rows). Below it the decode kernels serve it (chunks of up to 16 rows, split-K;
 * gate_up_down as one kernel from EXL3C4_GD_FUSE_MIN_T rows). The rule is the crossover measured on MI355X at the
 * decode layer's experts (512 experts, 2048 / 512, K = 4, softmax top-10): gate_up_down by the decode kernels against
 * the prefill kernels, us a launch, M tokens (3 x 400 launches, alternating on one box): M = 26: 107.7 / 126.4,
 * 28: 113.9 / 128.2, 32: 127.6 / 131.0, 36: 139.6 / 152.0, 40: 151.5 / 156.5, 44: 155.5 / 157.8, 48: 169.1 / 160.8,
 * 56: 186.8 / 186.0 (an earlier build: 64: 204 / 191, 128: 302 / 264, 256: 389 / 285, 409: 491 / 293): the rule's
 * M >= 45 (T >= 448) sits between 44 and 48. The reference serves M >= 17 by its GEMM rows (kernels/exl3r4d/rows.c:
 * 255-315, kernels/exl3r4d/prefill.c:61-76); here the decode kernels keep the band below the crossover. A function of
 * T, n_expert and the op's widths (never of the routing): the prefill GEMMs address a chunk's staged rows by 32-bit
 * byte offsets (2 x 111 x pitch + 64 < 2^32), so an input pitch past EXL3C4_PF_MAX_PITCH halves (the caller's x, the
 * rotated input's 2 x cols, h's rows / 2) keeps the decode kernels at any T. */
#ifndef EXL3C4_PF_MIN_T
#define EXL3C4_PF_MIN_T 64
#endif
#define EXL3C4_PF_MAX_PITCH (1 << 24)
int64_t exl3c4_prefill_min_rows(int64_t n_expert) {
    const int64_t r = (7 * (n_expert > 0 ? n_expert : 0) + 7) / 8;
    return r > EXL3C4_PF_MIN_T ? r : EXL3C4_PF_MIN_T;
}
static int prefill_path(const Exl3c4Op* o, int64_t T) {
    const int64_t pitch = o->x_pitch > 2 * max_cols(o) ? o->x_pitch : 2 * max_cols(o);
    return o->op != EXL3C4_PREP_GU && T >= exl3c4_prefill_min_rows(o->n_expert) && pitch <= EXL3C4_PF_MAX_PITCH &&
           max_rows(o) / 2 <= EXL3C4_PF_MAX_PITCH;
}

/* gate_up_down runs as one kernel at decode from this many sorted rows (the header's EXL3C4_GD_FUSE_MIN_T; a build
 * may move it to compare the two forms) */
#ifndef GD_FUSE_ROWS
#define GD_FUSE_ROWS EXL3C4_GD_FUSE_MIN_T
#endif

/* Below that, from GEPI_ROWS rows, gate_up_down forms h once a (row, 128-block) with gate_up's epilogue kernel (a wave
 * each, all in parallel) and down stages it as given; with fewer, down's workgroups form their chunk's h while staging
 * (one launch fewer, but every block's workgroup forms every row's h of its chunk, one row after another: slow when a
 * chunk holds many rows, which the host cannot see -- n_expert counts tables, not live experts). A build may move it. */
#ifndef GEPI_ROWS
#define GEPI_ROWS 2
#endif

typedef struct Carve {
    int     pf;                                   /* the prefill path */
    int     gd1;                                  /* gate_up_down as one kernel (decode path, T >= GD_FUSE_MIN_T) */
    int     h_gepi;                               /* gate_up_down, decode path below that (GEPI_ROWS): h by k_gepi */
    int64_t row_info, plan, xr, part, h, dacc, sync, total;
    int64_t T, part_pitch, dacc_pitch, xr_pitch, h_pitch, max_chunks;
    int     split_gu, gu_lds_pitch, dn_lds_pitch, chunk;
} Carve;

/* The scratch of one launch with T sorted rows, each region 256-B aligned.
 *   decode path:  [row_info | gate_up split-K partial sums | h (gate_up_down as one kernel) | down accumulations |
 *                  sync (gate_up_down as one kernel)]
 *   prefill path: [row_info | plan | rotated input | gate_up sums | h (gate_up_down) | down accumulations]
 * row_info: each row's owner (and, decode path, chunk rows), written by the first kernel for those after it. */
/* gate_up_down's down K (the op's dn_bits, else its bits). A mixed pair runs as one kernel for the mul1 codebook (the
 * instantiations k_gd carries); other codebooks take the three-kernel decode form, which every K has. */
static int dn_bits_of(const Exl3c4Op* o) { return o->dn_bits ? o->dn_bits : o->bits; }
static int gd_pair(const Exl3c4Op* o) { return dn_bits_of(o) == o->bits || o->codebook == EXL3C4_CB_MUL1; }

static void carve(const Exl3c4Op* o, int64_t T, Carve* k) {
    const int op = o->op;
    const int64_t rc = max_rows(o), xc = max_cols(o);
    memset(k, 0, sizeof *k);
    k->T = T;
    k->pf = prefill_path(o, T);
    k->chunk = chunk_for(o->M);
    int64_t off = 0;
    const int gu = op == EXL3C4_GATE_UP || op == EXL3C4_GU_DN;
    const int dn = op == EXL3C4_DOWN || op == EXL3C4_GU_DN;
    k->row_info = off;
    if (gu || (dn && k->pf)) off += ALIGN_UP(T * 8, 256);
    k->plan = off;
    if (k->pf) {
        k->max_chunks = T / EXL3C4_PF_ROWS_WIDE + (o->n_expert < T ? o->n_expert : T) + 1;   /* the smaller chunks */
        off += ALIGN_UP(4 * EXL3C4_PF_PLAN_HDR + 24 * k->max_chunks, 256);   /* entries, then two chunk orders */
    }
    k->xr = off;
    if (k->pf) {
        if ((op == EXL3C4_GATE_UP && !o->a_rot) || op == EXL3C4_GU_DN) k->xr_pitch = 2 * xc;
        else if (op == EXL3C4_DOWN && !o->h_rot) k->xr_pitch = xc;
        off += ALIGN_UP(T * k->xr_pitch * 2, 256);
    }
    k->part = off;
    if (gu) {
        int64_t nb_min = INT64_MAX, nb_max = 0;
        for (int c = 0; c < o->n_class; ++c) {
            const int64_t nb = o->cls[c].cols / 128;
            if (nb < nb_min) nb_min = nb;
            if (nb > nb_max) nb_max = nb;
        }
        int s = 1;
        if (!k->pf) {   /* split-K from T, M and the geometry: ksplit_for */
            s = ksplit_for(chunk_bound(T, o->n_expert, k->chunk), rc / 128, nb_min, nb_max, k->chunk);
            k->gu_lds_pitch = (int)(((nb_max + s - 1) / s) * 128 + 8);
        }
        k->split_gu = s;
        k->part_pitch = rc;
        off += ALIGN_UP(s * T * rc * 4, 256);
    }
    k->gd1 = op == EXL3C4_GU_DN && !k->pf && T >= GD_FUSE_ROWS && gd_pair(o);
    k->h_gepi = op == EXL3C4_GU_DN && !k->pf && !k->gd1 && T >= GEPI_ROWS;
    k->h = off;
    if ((k->pf || k->gd1 || k->h_gepi) && op == EXL3C4_GU_DN) {
        k->h_pitch = rc / 2;
        off += ALIGN_UP(T * k->h_pitch * 2, 256);
    }
    k->dacc = off;
    if (dn) {
        /* down's geometry: its own classes, or gate_up_down's [cols, rows / 2] */
        int64_t nmax = 0, kmax = 0;
        for (int c = 0; c < o->n_class; ++c) {
            const int64_t r = op == EXL3C4_DOWN ? o->cls[c].rows : o->cls[c].cols;
            const int64_t kk = op == EXL3C4_DOWN ? o->cls[c].cols : o->cls[c].rows / 2;
            if (r > nmax) nmax = r;
            if (kk > kmax) kmax = kk;
        }
        k->dacc_pitch = nmax;
        k->dn_lds_pitch = (int)(kmax + 8);     /* padded: the 16 staged rows start in different LDS banks */
        off += ALIGN_UP(T * nmax * 4, 256);
    }
    k->sync = off;
    if (k->gd1) off += (T + 1) * EXL3C4_SYNC_STRIDE * 4;   /* the status word, a counter a row (256 B each) */
    k->total = off;
}

/* ------------------------------------------------------------------ refusals */

static int class_ok(const Exl3c4Op* o, const Exl3c4Class* c, int gate_up_geom, int need_suh1, int need_dn_suh,
                    int need_codes) {
    if (c->cols <= 0 || c->cols % 128) return EXL3C4_E_SHAPE;
    if (o->op != EXL3C4_PREP_GU && (c->rows <= 0 || c->rows % (gate_up_geom ? 256 : 128))) return EXL3C4_E_SHAPE;
    if (!c->suh || (need_suh1 && !c->suh1) || (need_dn_suh && !c->dn_suh)) return EXL3C4_E_INVAL;
    if (need_codes && (!c->codes || !c->svh)) return EXL3C4_E_INVAL;
    if (c->codes_stride < 0 || c->suh_stride < 0 || c->suh1_stride < 0 || c->svh_stride < 0 || c->dn_suh_stride < 0)
        return EXL3C4_E_STRIDE;
    if (need_codes && c->codes_stride && (c->codes_stride % 4 || (uintptr_t)c->codes % 4)) return EXL3C4_E_ALIGN;
    if ((c->suh_stride | c->suh1_stride | c->svh_stride | c->dn_suh_stride) & 1) return EXL3C4_E_ALIGN;
    if (need_codes && c->codes_stride && c->codes_stride < exl3c4_record_bytes(c->rows, c->cols, o->bits))
        return EXL3C4_E_STRIDE;
    /* a stacked scale table's entries hold the whole vector: suh / suh1 [cols], svh [rows], dn_suh [rows / 2] */
    if ((c->suh_stride && c->suh_stride < 2 * (int64_t)c->cols) ||
        (need_suh1 && c->suh1_stride && c->suh1_stride < 2 * (int64_t)c->cols) ||
        (need_codes && c->svh_stride && c->svh_stride < 2 * (int64_t)c->rows) ||
        (need_dn_suh && c->dn_suh_stride && c->dn_suh_stride < (int64_t)c->rows))
        return EXL3C4_E_STRIDE;
    if (c->codes_stride > INT32_MAX || c->suh_stride > INT32_MAX || c->suh1_stride > INT32_MAX ||
        c->svh_stride > INT32_MAX || c->dn_suh_stride > INT32_MAX)
        return EXL3C4_E_STRIDE;
    return EXL3C4_OK;
}

static int check(const Exl3c4Op* o) {
    const int op = o->op;
    if (op < EXL3C4_DOWN || op > EXL3C4_GU_DN) return EXL3C4_E_INVAL;
    if (!o->x || !o->y || !o->sorted_tok || !o->expert_offset) return EXL3C4_E_INVAL;
    if (o->n_class != 1 && o->n_class != 2 && o->n_class != 4) return EXL3C4_E_INVAL;
    if ((o->h_rot != 0 && o->h_rot != 1) || (o->a_rot != 0 && o->a_rot != 1)) return EXL3C4_E_INVAL;
    if (op != EXL3C4_GATE_UP && o->a_rot) return EXL3C4_E_INVAL;
    if (o->bits < 2 || o->bits > 8) return EXL3C4_E_DTYPE;
    if (o->dn_bits && (o->dn_bits < 2 || o->dn_bits > 8)) return EXL3C4_E_DTYPE;
    if (o->dn_bits && o->dn_bits != o->bits && op != EXL3C4_GU_DN) return EXL3C4_E_INVAL;
    if (op != EXL3C4_PREP_GU && (o->codebook < EXL3C4_CB_3INST || o->codebook > EXL3C4_CB_MUL1)) return EXL3C4_E_DTYPE;
    if (o->M < 1 || o->n_expert < 1 || o->top_k < 1 || o->T < 0) return EXL3C4_E_SHAPE;
    if (o->n_expert > 65536) return EXL3C4_E_SHAPE;
    const int gu = is_gate_up(op);
    for (int c = 0; c < o->n_class; ++c) {
        const int need_dn = (op == EXL3C4_GATE_UP && o->h_rot) || op == EXL3C4_GU_DN;
        const int rc = class_ok(o, &o->cls[c], gu, gu, need_dn, op != EXL3C4_PREP_GU);
        if (rc) return rc;
        if (op == EXL3C4_GU_DN) {
            const Exl3c4Class* d = &o->dn[c];
            if (!d->codes || !d->svh) return EXL3C4_E_INVAL;
            if (d->rows != o->cls[c].cols || d->cols != o->cls[c].rows / 2) return EXL3C4_E_SHAPE;
            if (d->codes_stride < 0 || d->svh_stride < 0) return EXL3C4_E_STRIDE;
            if (d->codes_stride && (d->codes_stride % 4 || (uintptr_t)d->codes % 4)) return EXL3C4_E_ALIGN;
            if (d->svh_stride & 1) return EXL3C4_E_ALIGN;
            /* down's [cols, rows / 2] weight: a stacked entry holds its record, svh [cols] */
            if (d->codes_stride && d->codes_stride < exl3c4_record_bytes(d->rows, d->cols, dn_bits_of(o)))
                return EXL3C4_E_STRIDE;
            if (d->svh_stride && d->svh_stride < 2 * (int64_t)d->rows) return EXL3C4_E_STRIDE;
            if (d->codes_stride > INT32_MAX || d->svh_stride > INT32_MAX) return EXL3C4_E_STRIDE;
        }
    }
    /* down stages a chunk's 16 input rows in LDS: at most 1536 columns (49 KiB) */
    for (int c = 0; c < o->n_class; ++c) {
        const int64_t kdn = op == EXL3C4_DOWN ? o->cls[c].cols : op == EXL3C4_GU_DN ? o->cls[c].rows / 2 : 0;
        if (kdn > 1536) return EXL3C4_E_UNSUPPORTED;
    }
    /* the input: token rows (f16 or bf16) or sorted rows (f16) */
    const int token_rows = (op == EXL3C4_GATE_UP && !o->a_rot) || op == EXL3C4_PREP_GU || op == EXL3C4_GU_DN;
    if (o->x_dtype != EXL3C4_F16 && !(token_rows && o->x_dtype == EXL3C4_BF16)) return EXL3C4_E_DTYPE;
    const int64_t xc = max_cols(o), rc = max_rows(o);
    const int64_t need_x = op == EXL3C4_GATE_UP && o->a_rot ? 2 * xc : xc;
    if (o->x_cols < need_x) return EXL3C4_E_SHAPE;
    if (o->x_pitch < o->x_cols || o->x_pitch > INT32_MAX) return EXL3C4_E_STRIDE;
    if (!token_rows && o->x_rows < o->T) return EXL3C4_E_SHAPE;
    if (token_rows && o->x_rows < 1 && o->T > 0) return EXL3C4_E_SHAPE;
    const int gemm_reads_x = (op == EXL3C4_GATE_UP && o->a_rot) || (op == EXL3C4_DOWN && o->h_rot);
    if (gemm_reads_x && ((uintptr_t)o->x % 16 || (o->x_pitch * 2) % 16)) return EXL3C4_E_ALIGN;
    if ((uintptr_t)o->x % 2) return EXL3C4_E_ALIGN;
    /* the output: exactly the op's width */
    const int64_t want = op == EXL3C4_PREP_GU ? 2 * xc : op == EXL3C4_GATE_UP ? rc / 2 : op == EXL3C4_GU_DN ? xc : rc;
    if (o->y_cols != want) return EXL3C4_E_SHAPE;
    if (o->y_pitch < o->y_cols || o->y_pitch > INT32_MAX) return EXL3C4_E_STRIDE;
    if ((uintptr_t)o->y % 2) return EXL3C4_E_ALIGN;
    return EXL3C4_OK;
}

/* The scratch a launch of any T' in [1, Ttop] sorted rows needs: the largest carve over them. The carve is not
 * monotone in T: the decode path's split-K count grows as T shrinks (so its partial sums s T' N can grow), and the
 * prefill path's regions replace the decode path's at its threshold. A caller that sizes scratch once, at the band top
 * (docs/STEP0.md:142-146), must be able to launch every smaller batch in it. */
static int64_t carve_max(const Exl3c4Op* o, int64_t Ttop) {
    int64_t m = 0;
    Carve k;
    for (int64_t t = 1; t <= Ttop; ++t) {
        carve(o, t, &k);
        if (k.total > m) m = k.total;
    }
    return m;
}

int64_t exl3c4_scratch_bytes(const Exl3c4Op* o) {
    Exl3c4Op q;
    int rc;
    if (!o) return EXL3C4_E_INVAL;
    q = *o;
    q.T = o->M * o->top_k > o->T ? o->M * o->top_k : o->T;
    if (q.x_rows < q.T) q.x_rows = q.T;   /* sized from the geometry: a sorted-row input as long as the band top */
    if ((rc = check(&q)) != EXL3C4_OK) return rc;
    return carve_max(&q, q.T);
}

int64_t exl3c4_launch_scratch_bytes(const Exl3c4Op* o) {
    int rc;
    if (!o) return EXL3C4_E_INVAL;
    if ((rc = check(o)) != EXL3C4_OK) return rc;
    Carve k;
    carve(o, o->T, &k);
    return k.total;
}

int64_t exl3c4_scratch_bytes_geom(int32_t op, int32_t n_class, const int32_t* rows, const int32_t* cols, int64_t M,
                                  int64_t top_k, int64_t n_expert) {
    Exl3c4Op q;
    Carve k;
    if (op < EXL3C4_DOWN || op > EXL3C4_GU_DN || !rows || !cols) return EXL3C4_E_INVAL;
    if (n_class != 1 && n_class != 2 && n_class != 4) return EXL3C4_E_INVAL;
    if (M < 1 || top_k < 1 || n_expert < 1 || n_expert > 65536) return EXL3C4_E_SHAPE;
    memset(&q, 0, sizeof q);
    q.op = op;
    q.n_class = n_class;
    q.M = M;
    q.top_k = top_k;
    q.n_expert = n_expert;
    for (int c = 0; c < n_class; ++c) {
        if (cols[c] <= 0 || cols[c] % 128) return EXL3C4_E_SHAPE;
        if (op != EXL3C4_PREP_GU && (rows[c] <= 0 || rows[c] % (is_gate_up(op) ? 256 : 128))) return EXL3C4_E_SHAPE;
        if ((op == EXL3C4_DOWN ? cols[c] : op == EXL3C4_GU_DN ? rows[c] / 2 : 0) > 1536) return EXL3C4_E_UNSUPPORTED;
        q.cls[c].rows = rows[c];
        q.cls[c].cols = cols[c];
    }
    (void)k;
    return carve_max(&q, M * top_k);
}

/* ------------------------------------------------------------------ the launch */

/* The classes as the kernels read them: every plane of class c of the op (gate_up_down: gate_up's, and down's codes
 * and svh as dn_codes / dn_svh). check() has bounded every stride to 32 bits. */
static void dev_classes(const Exl3c4Op* o, Exl3c4Launch* a) {
    for (int c = 0; c < o->n_class; ++c) {
        const Exl3c4Class* g = &o->cls[c];
        Exl3c4DevClass* d = &a->cls[c];
        d->codes = g->codes;
        d->suh = g->suh;
        d->suh1 = g->suh1;
        d->svh = g->svh;
        d->dn_suh = g->dn_suh;
        d->codes_s = (int32_t)g->codes_stride;
        d->suh_s = (int32_t)g->suh_stride;
        d->suh1_s = (int32_t)g->suh1_stride;
        d->svh_s = (int32_t)g->svh_stride;
        d->dn_suh_s = (int32_t)g->dn_suh_stride;
        d->rows = g->rows;
        d->cols = g->cols;
        if (o->op == EXL3C4_GU_DN) {
            d->dn_codes = o->dn[c].codes;
            d->dn_svh = o->dn[c].svh;
            d->dn_codes_s = (int32_t)o->dn[c].codes_stride;
            d->dn_svh_s = (int32_t)o->dn[c].svh_stride;
        }
    }
}

static void base_args(const Exl3c4Op* o, const Carve* k, char* s, Exl3c4Launch* a) {
    memset(a, 0, sizeof *a);
    dev_classes(o, a);
    a->sorted = o->sorted_tok;
    a->off = o->expert_offset;
    a->part = (float*)(s + k->part);
    a->part_pitch = (int32_t)k->part_pitch;
    a->T = (int32_t)o->T;
    a->n_expert = (int32_t)o->n_expert;
    a->top_k = (int32_t)o->top_k;
    a->n_class = o->n_class;
    a->bits = (int16_t)o->bits;
    a->dn_bits = (int16_t)dn_bits_of(o);
    a->codebook = o->codebook;
    a->x = o->x;
    a->x_pitch = (int32_t)o->x_pitch;
    a->x_dtype = o->x_dtype;
    a->x_rows = (int32_t)o->x_rows;
    a->x_cols_max = (int32_t)max_cols(o);
    a->y = o->y;
    a->y_pitch = (int32_t)o->y_pitch;
    a->y_cols = (int32_t)o->y_cols;
    a->blk_per_wave = 1;
    a->chunk_rows = k->chunk;
}

/* How a launch runs: the events of a timed launch go to exactly one kernel of the sequence; keep_sums has the
 * prefill GEMMs also write their f32 sums to scratch (exl3c4_launch_checked); ctr: gate_up_down's counter block from
 * the caller (exl3c4_launch_ctr), or null; gx: moe_gather riding in gate_up_down's single kernel
 * (exl3c4_launch_gather), or null; fail: a host-visible flag the single kernel sets when a wait gives up, or null. */
typedef struct {
    const float*   w;
    const int32_t* row_of;
    void*          out;
    int64_t        out_pitch;
} Gather;
typedef struct Ctx {
    int           kernel;
    void *        ev0, *ev1;
    int           keep_sums;
    int32_t*      ctr;
    const Gather* gx;
    int32_t*      fail;
} Ctx;
#define EV(k) (t->kernel == (k) ? t->ev0 : NULL), (t->kernel == (k) ? t->ev1 : NULL)

/* The prefill path: plan; the input rotation into scratch (unless the input arrives rotated); gate_up's GEMM and its
 * epilogue (into y, or into h for gate_up_down); down's GEMM with its epilogue; the rows no run holds zeroed. */
static int launch_prefill(const Exl3c4Op* o, const Carve* k, char* s, void* stream, const Ctx* t) {
    const int op = o->op;
    int rc;
    Exl3c4Launch p;
    base_args(o, k, s, &p);
    p.keep_sums = t->keep_sums;
    p.row_info = (int32_t*)(s + k->row_info);
    p.plan = (int32_t*)(s + k->plan);
    p.max_chunks = (int32_t)k->max_chunks;

    const void* gin = o->x;                       /* gate_up's GEMM input: xr */
    int64_t gin_pitch = o->x_pitch;
    const void* din = o->x;                       /* down's GEMM input: h, rotated */
    int64_t din_pitch = o->x_pitch;
    if (k->xr_pitch) {                            /* the rotation, its launch's last workgroup planning beside it */
        Exl3c4Launch r = p;
        r.y = s + k->xr;
        r.y_pitch = (int32_t)k->xr_pitch;
        r.h_from_gu = op == EXL3C4_DOWN ? 1 : 2;  /* halves a row */
        if ((rc = exl3c4_dev_rot(&r, stream, EV(EXL3C4_K_PREP))) != 0) return rc;
        if (op == EXL3C4_DOWN) { din = s + k->xr; din_pitch = k->xr_pitch; }
        else { gin = s + k->xr; gin_pitch = k->xr_pitch; }
    } else if ((rc = exl3c4_dev_plan(&p, stream, EV(EXL3C4_K_PREP))) != 0) {
        return rc;
    }
    if (op == EXL3C4_GATE_UP || op == EXL3C4_GU_DN) {
        Exl3c4Launch a = p;
        a.x = gin;
        a.x_pitch = (int32_t)gin_pitch;
        a.ksplit = 1;
        a.n_grp = (int32_t)(max_rows(o) / 128);
        a.h_rot = op == EXL3C4_GU_DN ? 1 : o->h_rot;
        if (op == EXL3C4_GU_DN) { a.y = s + k->h; a.y_pitch = (int32_t)k->h_pitch; a.nblk = (int32_t)(k->h_pitch / 128); }
        else a.nblk = (int32_t)(o->y_cols / 128);
        /* the GEMM with its epilogue: h (rotated for down when h_rot) for every row a chunk holds; gate_up alone
         * also zeroes the rows no run holds, in workgroups after the GEMM's */
        a.tail_from = op == EXL3C4_GATE_UP;
        if ((rc = exl3c4_dev_gu_pf(&a, stream, EV(EXL3C4_K_GATE_UP))) != 0) return rc;
        if (op == EXL3C4_GATE_UP) return EXL3C4_OK;
        din = s + k->h;
        din_pitch = k->h_pitch;
    }
    Exl3c4Launch d = p;
    d.dn_gd = op == EXL3C4_GU_DN;                 /* gate_up_down: down's planes of gate_up's classes */
    d.x = din;
    d.x_pitch = (int32_t)din_pitch;
    d.nblk = (int32_t)(o->y_cols / 128);
    d.dacc = (float*)(s + k->dacc);
    d.dacc_pitch = (int32_t)k->dacc_pitch;
    d.tail_from = 1;                              /* and the rows no run holds, zeroed after the GEMM's workgroups */
    return exl3c4_dev_dn_pf(&d, stream, EV(EXL3C4_K_DOWN));
}

/* gate_up_down at decode as one kernel: the row counters and status zeroed (or the caller's zeroed block taken), then
 * k_gd (gate_up units, then down units waiting on their row's counter; the row's last down unit zeroes its counters),
 * with moe_gather inside when asked (exl3c4_launch_gather). */
static int launch_gd1(const Exl3c4Op* o, const Carve* k, char* s, void* stream, const Ctx* t) {
    int rc;
    Exl3c4Launch g;
    base_args(o, k, s, &g);
    g.dn_gd = 1;
    g.h_from_gu = 1;
    g.ksplit = k->split_gu;
    g.ksplit_log2 = log2i(k->split_gu);
    g.n_grp = (int32_t)(max_rows(o) / 128);
    g.lds_pitch_gu = k->gu_lds_pitch;
    g.lds_pitch = k->dn_lds_pitch;
    g.nblk = (int32_t)(o->y_cols / 128);
    g.dacc = (float*)(s + k->dacc);
    g.dacc_pitch = (int32_t)k->dacc_pitch;
    g.hbuf = (uint16_t*)(s + k->h);
    g.hbuf_pitch = (int32_t)k->h_pitch;
    g.fail = t->fail;
    if (t->ctr) {                                 /* the caller's counter block: zero, and left zero */
        g.sync = t->ctr;
    } else {
        g.sync = (int32_t*)(s + k->sync);
        if ((rc = exl3c4_dev_fill(g.sync, (o->T + 1) * EXL3C4_SYNC_STRIDE, stream)) != 0) return rc;
    }
    if (t->gx) {                                  /* only with the caller's block: the token counters follow the rows' */
        g.g_w = t->gx->w;
        g.g_row_of = t->gx->row_of;
        g.g_out = (uint16_t*)t->gx->out;
        g.g_out_pitch = (int32_t)t->gx->out_pitch;
        g.g_ntok = (int32_t)o->M;
        g.g_ctr = t->ctr + (o->T + 1) * EXL3C4_SYNC_STRIDE;
    }
    return exl3c4_dev_gd(&g, stream, EV(EXL3C4_K_GATE_UP_DOWN));
}

/* The kernels a launch runs (for exl3c4_launch_timed). */
static int runs_kernel(const Exl3c4Op* o, const Carve* k, int kernel) {
    const int op = o->op;
    if (op == EXL3C4_PREP_GU) return kernel == EXL3C4_K_PREP;
    if (k->pf) {
        if (kernel == EXL3C4_K_PREP) return 1;                   /* the plan */
        if (kernel == EXL3C4_K_GATE_UP) return op != EXL3C4_DOWN;
        return kernel == EXL3C4_K_DOWN && op != EXL3C4_GATE_UP;
    }
    if (k->gd1) return kernel == EXL3C4_K_GATE_UP_DOWN;
    switch (op) {
    case EXL3C4_GATE_UP: return kernel == EXL3C4_K_GATE_UP || kernel == EXL3C4_K_EPI_GU;
    case EXL3C4_DOWN:    return kernel == EXL3C4_K_DOWN;
    default:             return kernel == EXL3C4_K_GATE_UP || kernel == EXL3C4_K_DOWN ||
                                (k->h_gepi && kernel == EXL3C4_K_EPI_GU);
    }
}

/* The launches of each op on the stream. Decode (fewer sorted rows than exl3c4_prefill_min_rows: prefill_path) has no
 * planning pass: every workgroup finds its rows' expert itself.
 *   prep_gu       the input rotation
 *   gate_up       its GEMM (input rotation staged inside), then its epilogue
 *   down          its GEMM, whose workgroups stage (and rotate) their rows and finish their output blocks
 *   gate_up_down  gate_up's GEMM, then down's, whose workgroups build h from gate_up's partial sums; from
 *                 GD_FUSE_MIN_T rows both GEMMs in one kernel (launch_gd1)
 * Prefill (launch_prefill) plans 64-row chunks of one expert first and runs one GEMM kernel a projection. */
static int launch_impl(const Exl3c4Op* o, void* scratch, int64_t scratch_bytes, void* stream, const Ctx* t) {
    int rc;
    if (!o) return EXL3C4_E_INVAL;
    if ((rc = check(o)) != EXL3C4_OK) return rc;
    Carve k;
    carve(o, o->T, &k);
    if (k.total > 0 && (!scratch || scratch_bytes < k.total || (uintptr_t)scratch % 256)) return EXL3C4_E_SCRATCH;
    if (o->T == 0) return EXL3C4_OK;
    char* s = (char*)scratch;
    const int op = o->op;

    if (op == EXL3C4_PREP_GU) {
        Exl3c4Launch f;
        base_args(o, &k, s, &f);
        return exl3c4_dev_prep(&f, stream, EV(EXL3C4_K_PREP));
    }

    if (k.pf) return launch_prefill(o, &k, s, stream, t);
    if (k.gd1) return launch_gd1(o, &k, s, stream, t);

    if (op == EXL3C4_GATE_UP || op == EXL3C4_GU_DN) {
        Exl3c4Launch a;
        base_args(o, &k, s, &a);
        a.row_info = (int32_t*)(s + k.row_info);
        a.a_rot = op == EXL3C4_GATE_UP ? o->a_rot : 0;
        a.h_rot = o->h_rot;
        a.ksplit = k.split_gu;
        a.ksplit_log2 = log2i(k.split_gu);
        a.n_grp = (int32_t)(max_rows(o) / 128);
        a.lds_pitch = k.gu_lds_pitch;
        a.nblk = (int32_t)(o->y_cols / 128);
        if ((rc = exl3c4_dev_gu(&a, stream, EV(EXL3C4_K_GATE_UP))) != 0) return rc;
        if (op == EXL3C4_GATE_UP) return exl3c4_dev_gepi(&a, stream, EV(EXL3C4_K_EPI_GU));
        if (k.h_gepi) {                              /* h (rotated for down) into scratch, a wave a (row, block) */
            Exl3c4Launch e = a;
            e.h_rot = 1;
            e.y = s + k.h;
            e.y_pitch = (int32_t)k.h_pitch;
            e.nblk = (int32_t)(max_rows(o) / 256);
            if ((rc = exl3c4_dev_gepi(&e, stream, EV(EXL3C4_K_EPI_GU))) != 0) return rc;
        }
    }

    /* down: its own classes, or gate_up_down's [cols, rows / 2] over h with suh = gate_up's dn_suh
     * (include/exl3_abi.h:751-800; h crosses rotated) */
    Exl3c4Launch d;
    base_args(o, &k, s, &d);
    d.dn_gd = op == EXL3C4_GU_DN;
    if (op == EXL3C4_GU_DN && k.h_gepi) {
        d.row_info = (int32_t*)(s + k.row_info);     /* written by gate_up's GEMM */
        d.x = s + k.h;                               /* h, rotated: staged as given */
        d.x_pitch = (int32_t)k.h_pitch;
        d.x_rows = (int32_t)o->T;
        d.h_rot = 1;
    } else if (op == EXL3C4_GU_DN) {
        d.h_from_gu = 1;
        d.row_info = (int32_t*)(s + k.row_info);     /* written by gate_up's GEMM */
        d.ksplit = k.split_gu;                       /* the gate_up partial sums it reads */
    } else {
        d.h_rot = o->h_rot;
    }
    d.nblk = (int32_t)(o->y_cols / 128);
    d.lds_pitch = k.dn_lds_pitch;
    d.dacc = (float*)(s + k.dacc);
    d.dacc_pitch = (int32_t)k.dacc_pitch;
    return exl3c4_dev_dn(&d, stream, EV(EXL3C4_K_DOWN));
}

int exl3c4_launch(const Exl3c4Op* o, void* scratch, int64_t scratch_bytes, void* stream) {
    const Ctx t = { -1, NULL, NULL, 0, NULL, NULL, NULL };
    return launch_impl(o, scratch, scratch_bytes, stream, &t);
}

int exl3c4_launch_checked(const Exl3c4Op* o, void* scratch, int64_t scratch_bytes, void* stream) {
    const Ctx t = { -1, NULL, NULL, 1, NULL, NULL, NULL };
    return launch_impl(o, scratch, scratch_bytes, stream, &t);
}

int64_t exl3c4_ctr_bytes(const Exl3c4Op* o) {
    Exl3c4Op q;
    int rc;
    if (!o) return EXL3C4_E_INVAL;
    q = *o;
    q.T = o->M * o->top_k > o->T ? o->M * o->top_k : o->T;
    if (q.x_rows < q.T) q.x_rows = q.T;
    if ((rc = check(&q)) != EXL3C4_OK) return rc;
    /* the status word and a counter a row, then a counter line a token (exl3c4_launch_gather) */
    return q.op == EXL3C4_GU_DN ? ALIGN_UP((q.T + 1 + o->M) * EXL3C4_SYNC_STRIDE * 4, 256) : 0;
}

int exl3c4_launch_inst(const Exl3c4Op* o, void* scratch, int64_t scratch_bytes, void* stream, void* ctr,
                       int64_t ctr_bytes, int32_t* fail) {
    int rc;
    if (!o) return EXL3C4_E_INVAL;
    if ((rc = check(o)) != EXL3C4_OK) return rc;
    Carve k;
    carve(o, o->T, &k);
    if (k.gd1 && ctr && (ctr_bytes < (o->T + 1) * EXL3C4_SYNC_STRIDE * 4 || (uintptr_t)ctr % 256))
        return EXL3C4_E_SCRATCH;
    const Ctx t = { -1, NULL, NULL, 0, k.gd1 ? (int32_t*)ctr : NULL, NULL, fail };
    return launch_impl(o, scratch, scratch_bytes, stream, &t);
}

int exl3c4_launch_ctr(const Exl3c4Op* o, void* scratch, int64_t scratch_bytes, void* stream, void* ctr,
                      int64_t ctr_bytes) {
    return exl3c4_launch_inst(o, scratch, scratch_bytes, stream, ctr, ctr_bytes, NULL);
}

int exl3c4_launch_gather(const Exl3c4Op* o, void* scratch, int64_t scratch_bytes, void* stream, void* ctr,
                         int64_t ctr_bytes, const float* expert_w, const int32_t* row_of, void* out, int64_t out_pitch) {
    int rc;
    if (!o) return EXL3C4_E_INVAL;
    if ((rc = check(o)) != EXL3C4_OK) return rc;
    if (o->op != EXL3C4_GU_DN && o->op != EXL3C4_DOWN) return EXL3C4_E_INVAL;   /* y must be down's bf16 output */
    if (!expert_w || !row_of || !out) return EXL3C4_E_INVAL;
    if (out_pitch < o->y_cols || out_pitch > INT32_MAX) return EXL3C4_E_STRIDE;  /* exl3c4_moe_gather's refusals */
    if ((uintptr_t)o->y % 16 || (o->y_pitch * 2) % 16 || (uintptr_t)out % 16 || (out_pitch * 2) % 16 ||
        (uintptr_t)expert_w % 4 || (uintptr_t)row_of % 4)
        return EXL3C4_E_ALIGN;
    Carve k;
    carve(o, o->T, &k);
    const int fuse = k.gd1 && ctr && o->y_cols / 128 <= EXL3C4_SYNC_STRIDE;
    if (fuse && (ctr_bytes < (o->T + 1 + o->M) * EXL3C4_SYNC_STRIDE * 4 || (uintptr_t)ctr % 256))
        return EXL3C4_E_SCRATCH;
    if (k.gd1 && ctr && !fuse && (ctr_bytes < (o->T + 1) * EXL3C4_SYNC_STRIDE * 4 || (uintptr_t)ctr % 256))
        return EXL3C4_E_SCRATCH;
    const Gather gx = { expert_w, row_of, out, out_pitch };
    const Ctx tf = { -1, NULL, NULL, 0, (int32_t*)ctr, &gx, NULL };
    if (fuse) return launch_impl(o, scratch, scratch_bytes, stream, &tf);
    const Ctx t = { -1, NULL, NULL, 0, k.gd1 ? (int32_t*)ctr : NULL, NULL, NULL };
    if ((rc = launch_impl(o, scratch, scratch_bytes, stream, &t)) != EXL3C4_OK) return rc;
    return exl3c4_moe_gather(o->y, EXL3C4_BF16, o->y_pitch, expert_w, row_of, o->M, o->top_k, o->y_cols, out,
                             out_pitch, stream);
}

int exl3c4_launch_timed(const Exl3c4Op* o, void* scratch, int64_t scratch_bytes, void* stream, int32_t kernel,
                        void* ev_start, void* ev_stop) {
    int rc;
    if (!o || !ev_start || !ev_stop) return EXL3C4_E_INVAL;
    if ((rc = check(o)) != EXL3C4_OK) return rc;
    Carve k;
    carve(o, o->T, &k);
    if (!runs_kernel(o, &k, kernel)) return EXL3C4_E_INVAL;
    const Ctx t = { kernel, ev_start, ev_stop, 0, NULL, NULL, NULL };
    return launch_impl(o, scratch, scratch_bytes, stream, &t);
}

int exl3c4_scratch_partials(const Exl3c4Op* o, int32_t gemm, int64_t* offset, int64_t* pitch, int64_t* split_stride,
                            int32_t* splits) {
    int rc;
    if (!o || !offset || !pitch || !split_stride || !splits) return EXL3C4_E_INVAL;
    if ((rc = check(o)) != EXL3C4_OK) return rc;
    if (o->op == EXL3C4_PREP_GU || (gemm == 1 && o->op != EXL3C4_GU_DN) || gemm < 0 || gemm > 1) return EXL3C4_E_INVAL;
    Carve k;
    carve(o, o->T, &k);
    if (o->op == EXL3C4_DOWN || gemm == 1) {
        *offset = k.dacc;
        *pitch = k.dacc_pitch;
        *split_stride = k.T * k.dacc_pitch;
        *splits = 1;
    } else {
        *offset = k.part;
        *pitch = k.part_pitch;
        *split_stride = k.T * k.part_pitch;
        *splits = k.split_gu;
    }
    return EXL3C4_OK;
}

int exl3c4_scratch_status(const Exl3c4Op* o, int64_t* offset) {
    int rc;
    if (!o || !offset) return EXL3C4_E_INVAL;
    if ((rc = check(o)) != EXL3C4_OK) return rc;
    Carve k;
    carve(o, o->T, &k);
    if (!k.gd1) return EXL3C4_E_INVAL;
    *offset = k.sync;
    return EXL3C4_OK;
}

int exl3c4_dequant(const void* record, int32_t rows, int32_t cols, int32_t bits, int32_t codebook, void* w_hat,
                   int64_t w_pitch, void* stream) {
    if (!record || !w_hat) return EXL3C4_E_INVAL;
    if (bits < 1 || bits > 8 || codebook < EXL3C4_CB_3INST || codebook > EXL3C4_CB_MUL1) return EXL3C4_E_DTYPE;
    if (rows <= 0 || cols <= 0 || rows % EXL3C4_STRIP || cols % EXL3C4_KSTEP) return EXL3C4_E_SHAPE;
    if (w_pitch < cols) return EXL3C4_E_STRIDE;
    if ((uintptr_t)record % 4 || (uintptr_t)w_hat % 2) return EXL3C4_E_ALIGN;
    return exl3c4_dev_dequant(record, rows, cols, bits, codebook, w_hat, w_pitch, stream);
}

const char* exl3c4_build_target(void) { return "gfx950"; }
int         exl3c4_abi_version(void) { return EXL3C4_ABI_VERSION; }
