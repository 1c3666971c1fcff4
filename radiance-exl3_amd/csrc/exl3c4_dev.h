/* exl3c4_dev.h -- what the C host side (exl3c4_ops.c) hands the HIP side (exl3c4_dev.hip): one plain argument block,
 * passed by value to every kernel, and the extern "C" launchers. No radiance types, no torch types; a stream is a
 * hipStream_t carried as void*. The reference's counterpart is kernels/exl3r4d/exl3r4d_dev.h:29-109. */
#ifndef EXL3C4_DEV_H
#define EXL3C4_DEV_H

#include <stdint.h>

#include "exl3c4.h"

#ifdef __cplusplus
extern "C" {
#endif

/* Rows one MFMA row block holds: the most a chunk of an expert's run holds on the decode path (the GEMV's unit of
 * rows). A launch takes chunks of Exl3c4Launch.chunk_rows (a power of two up to this), its staged rows in LDS. */
#define EXL3C4_CHUNK_ROWS 16
/* Columns one wave's strip holds (two 16-column tiles) and k one step consumes (four 16-k tiles). */
#define EXL3C4_STRIP 32
#define EXL3C4_KSTEP 64
/* int32 words between two row counters of gate_up_down's single kernel (256 B: each counter its own cache line), and
 * where in a row's line the count of its down units past their wait sits */
#define EXL3C4_SYNC_STRIDE 64
#define EXL3C4_SYNC_DONE 32
/* Rows of one chunk on the prefill path at most: seven MFMA row tiles share each decoded step where a launch's K are
 * at most 4, six (EXL3C4_PF_ROWS_WIDE) at larger K. */
#define EXL3C4_PF_ROWS 112
#define EXL3C4_PF_ROWS_WIDE 96
/* The prefill plan: PF_PLAN_HDR int32s, then int4 {expert, row0, rows, 0} per chunk. Header: [0] the chunk count;
 * [PF_CUR + 32 (8 g + x)] (g = 0 gate_up, 1 down): XCD x's cursor over the last units of its range in that GEMM
 * (down deals none by cursor today), zeroed by the plan, each on its own 128-byte line;
 * [PF_SPAN] 1 when the rows the chunks hold are one span, [PF_SPAN + 1] its first row, [PF_SPAN + 2] its end (0: the
 * rows' owners are in row_info instead); [PF_XCD_GU + x], [PF_XCD_DN + x] (x = 0 .. 8): the first chunk of XCD x for
 * gate_up's and down's GEMM ([.. + 8] = the count). A chunk of t 16-row tiles costs about PF_W_GU + t (gate_up) and
 * PF_W_DN + t (down) units of workgroup time. */
#define EXL3C4_PF_PLAN_HDR (32 + 16 * 32)
#define EXL3C4_PF_SPAN 4
#define EXL3C4_PF_XCD_GU 8
#define EXL3C4_PF_XCD_DN 20
#define EXL3C4_PF_CUR 32
#define EXL3C4_PF_W_GU 10
#define EXL3C4_PF_W_DN 3

/* One class of experts as a kernel reads it: each plane's table -- a device pointer array when its stride is 0 (the
 * engine's form), else a stacked buffer with entry j at base + j * stride bytes -- and the class's weight geometry
 * [rows, cols]. The op's own weight is codes / suh / svh (with suh1 and dn_suh for gate_up); for gate_up_down the class
 * is gate_up's and dn_codes / dn_svh are down's planes, down's weight being [cols, rows / 2] with suh = dn_suh
 * (include/exl3_abi.h:751-800). */
typedef struct Exl3c4DevClass {
    const void* codes;
    const void* suh;
    const void* suh1;
    const void* svh;
    const void* dn_suh;
    const void* dn_codes;
    const void* dn_svh;
    int32_t     codes_s, suh_s, suh1_s, svh_s, dn_suh_s, dn_codes_s, dn_svh_s;   /* entry strides (bytes) */
    int32_t     rows, cols;
} Exl3c4DevClass;

/* The argument block every op kernel takes by value. The radiance engine dispatches a kernel only if its argument
 * segment -- these bytes plus any hidden argument HIP appends for a kernel that reads one (blockDim, gridDim, ...) --
 * fits its 768-byte slot (kernels/exl3r4d/exl3r4d_dev.h:5-6, tests/gpu/kernarg_check.sh): this block is 632 bytes
 * (EXL3C4_KERNARG_BYTES, checked at compile time) and no kernel that takes it reads a hidden argument. Hence the
 * 32-bit pitches and strides (the host refuses larger ones) and one class record serving both GEMMs of gate_up_down. */
#define EXL3C4_KERNARG_LIMIT 768
typedef struct Exl3c4Launch {
    Exl3c4DevClass cls[4];        /* the op's classes: class c holds experts e % n_class == c at entry e / n_class */
    const void*    x;             /* the input: token rows, or sorted rows (a_rot gate_up; down) */
    void*          y;             /* the op's output */
    float*         part;          /* gate_up's split-K partial sums [ksplit][T][part_pitch] */
    float*         dacc;          /* down's raw accumulations [T][dacc_pitch] */
    int32_t*       row_info;      /* [T][2]: the row's owner expert (-1: none), the chunk's rows where one starts */
    const int32_t* sorted;
    const int32_t* off;
    int32_t*       plan;          /* prefill: [0] chunk count, then int4 {expert, row0, rows, 0} per chunk */
    int32_t*       sync;          /* gate_up_down in one launch: a status word, then row i's counter at (i + 1) * SYNC_STRIDE */
    uint16_t*      hbuf;          /* gate_up_down in one launch: h (rotated, f16) of every chunk's rows [T][hbuf_pitch] */
    /* gate_up_down in one launch with moe_gather behind it (g_out non-null): out[t] = f16(sum over the token's slots
     * of expert_w x y[row_of]); token t's counter of 128-block b at g_ctr[t * SYNC_STRIDE + b] (zero, left zero) */
    const float*   g_w;
    const int32_t* g_row_of;
    uint16_t*      g_out;
    int32_t*       g_ctr;
    int32_t*       fail;          /* gate_up_down in one launch: also set to 1 when a wait gives up (host-visible), or null */
    int32_t        x_pitch, y_pitch, part_pitch, dacc_pitch, hbuf_pitch, g_out_pitch;   /* elements */
    int32_t        x_dtype, x_rows, x_cols_max;
    int32_t        T, n_expert, top_k, n_class;
    int16_t        bits, dn_bits;  /* gate_up's (and down's alone) K; down's K inside gate_up_down */
    int32_t        codebook;
    int32_t        h_rot;         /* gate_up: rotate h for down; down: the input is already rotated */
    int32_t        a_rot;         /* gate_up: the input is already rotated (sorted rows [T][2 C]) */
    int32_t        h_from_gu;     /* down: stage h from gate_up's partial sums (gate_up_down); k_rot: halves a row */
    int32_t        dn_gd;         /* down's weight is gate_up_down's (dn_codes / dn_svh / dn_suh of gate_up's class) */
    int32_t        ksplit, ksplit_log2;
    int32_t        n_grp;         /* gate_up: groups of four strips a row (the widest class's rows / 128) */
    int32_t        nblk;          /* epilogue / down: 128-column output blocks a row */
    int32_t        lds_pitch;     /* halves a staged input row in LDS */
    int32_t        lds_pitch_gu;  /* gate_up_down in one launch: gate_up's staged row pitch (lds_pitch is down's) */
    int32_t        y_cols;
    int32_t        max_chunks;
    int32_t        blk_per_wave;  /* gate_up's epilogue: 128-blocks of a row one wave takes */
    int32_t        keep_sums;     /* prefill: also leave the GEMMs' f32 sums in part / dacc (a checker's view) */
    int32_t        tail_from;     /* prefill GEMMs: nonzero asks for workgroups that zero the rows no run holds after
                                     the GEMM's (the launcher sets where they start) */
    int32_t        g_ntok;
    int32_t        chunk_rows;    /* decode path: rows a chunk holds at most (a power of two <= EXL3C4_CHUNK_ROWS) */
} Exl3c4Launch;
#define EXL3C4_KERNARG_BYTES 632

/* exl3c4_launch_ctr with a host-visible flag (`fail`, pinned host memory the device can write, or null) that the
 * single gate_up_down kernel sets to 1 when a wait gives up: what the plugin rows' instances hand over, so that a
 * later launch can report the failure without a synchronisation. Internal to the library. */
__attribute__((visibility("hidden"))) int exl3c4_launch_inst(const Exl3c4Op* o, void* scratch, int64_t scratch_bytes,
                                                             void* stream, void* ctr, int64_t ctr_bytes, int32_t* fail);

/* Each returns 0 or EXL3C4_E_DEVICE (a launch error). None allocates or synchronises. ev0 / ev1: hipEvent_t the
 * dispatch itself stamps at its start and end (hipExtLaunchKernelGGL), or null for a plain launch. */
int exl3c4_dev_prep(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_gu(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_gepi(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_dn(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
/* gate_up_down in one launch (k_gd): sync[0..T] zeroed first (exl3c4_dev_fill), then gate_up and down units */
int exl3c4_dev_gd(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_fill(int32_t* p, int64_t n, void* stream);
/* instance state (the plugin rows' init hooks): device memory zeroed once; pinned host memory the device writes */
void* exl3c4_dev_zalloc(int64_t bytes);
void  exl3c4_dev_free(void* p);
void* exl3c4_host_zalloc(int64_t bytes);
void  exl3c4_host_free(void* p);
/* the prefill path */
int exl3c4_dev_plan(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_rot(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_gu_pf(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_dn_pf(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
/* the routing (exl3c4_route.hip) */
int exl3c4_dev_router(const void* logits, int32_t dtype, int64_t n_tok, int32_t n_expert, int64_t pitch, int32_t top_k,
                      int32_t renorm, int32_t* ids, float* w, void* stream);
int exl3c4_dev_scatter(const int32_t* ids, int64_t T, int64_t base, int32_t n_expert, int32_t* sorted, int32_t* off,
                       int32_t* count, int32_t* row_of, void* stream);
int exl3c4_dev_route_scatter(const void* logits, int32_t dtype, int32_t n_tok, int32_t n_expert, int64_t pitch,
                             int32_t top_k, int32_t renorm, int32_t* ids, float* w, int32_t* sorted, int32_t* off,
                             int32_t* count, int32_t* row_of, void* stream);
int exl3c4_dev_gather(const void* y, int32_t y_dtype, int64_t y_pitch, const float* w, const int32_t* row_of,
                      int64_t n_tok, int32_t top_k, int64_t cols, void* out, int64_t out_pitch, void* stream);
int exl3c4_dev_dequant(const void* record, int32_t rows, int32_t cols, int32_t bits, int32_t codebook, void* w_hat,
                       int64_t w_pitch, void* stream);

#ifdef __cplusplus
}
#endif

#endif
