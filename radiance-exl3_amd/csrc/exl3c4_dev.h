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

/* Rows one MFMA row block holds: a chunk of an expert's run (the decode GEMV's unit of rows). */
#define EXL3C4_CHUNK_ROWS 16
/* Columns one wave's strip holds (two 16-column tiles) and k one step consumes (four 16-k tiles). */
#define EXL3C4_STRIP 32
#define EXL3C4_KSTEP 64

typedef struct Exl3c4Launch {
    Exl3c4Class    cls[4];        /* the GEMM's weight classes (gate_up's, or down's); prep: the scale source */
    const void*    x;             /* prep source: token rows (gate_up) or h (down h_rot 0) */
    int64_t        x_pitch;
    const void*    a;             /* GEMM A: xr [T][2 C] (gate_up) or h / rotated h [T][C] (down), f16 */
    int64_t        a_pitch;
    void*          y;             /* epilogue / prep output */
    int64_t        y_pitch;
    float*         part;          /* split-K partial sums [ksplit][T][part_pitch] */
    int64_t        part_pitch, part_split;
    int32_t*       plan;          /* [0] chunk count, then int4 {expert, row0, rows, 0} per chunk */
    const int32_t* sorted;
    const int32_t* off;
    int32_t        x_dtype, x_rows;
    int32_t        T, n_expert, top_k, n_class;
    int32_t        h_rot, ksplit, ksplit_log2, max_chunks, max_strips;
    int32_t        y_cols, gate_up, prep_mode, bits, codebook;
    int32_t        x_cols_max;    /* prep: the widest class's input width */
    int32_t        nblk;          /* epilogue: 128-column output blocks a row */
    int32_t*       ctr;           /* front: counters to zero (none at present) */
    int32_t        ctr_n;
    int32_t        a_perm;        /* GEMM: the activation rows are stored permuted */
    int32_t        out_perm;      /* epilogue: store the output rows permuted (gate_up_down's h) */
    int32_t        prep_perm;     /* front: store xr permuted */
    int32_t        prep_halves;   /* front: halves a row to rotate (2 gate_up, 1 down, 0 none) */
    int32_t        do_plan;       /* front: workgroup 0 plans the chunks */
    void*          z;             /* front: the output whose dead rows and class tails are zeroed */
    int64_t        z_pitch;
    int32_t        z_cols, zero_waves;
    int32_t        z_width[4];    /* a class's written width of z */
    Exl3c4Class    gcls[4];       /* down fused after gate_up: gate_up's classes (svh, dn_suh, its partial sums) */
    int32_t        h_from_gu;     /* down: stage h from gate_up's partial sums (gate_up_down) instead of `a` */
    int32_t        lds_pitch;     /* down: halves a staged input row */
    float*         dacc;          /* down: its raw accumulations [T][dacc_pitch] */
    int64_t        dacc_pitch;
} Exl3c4Launch;

/* prep modes */
enum { EXL3C4_PREP_GU_SCRATCH = 0, EXL3C4_PREP_GU_OP = 1, EXL3C4_PREP_DN = 2 };

/* Each returns 0 or EXL3C4_E_DEVICE (a launch error). None allocates or synchronises. ev0 / ev1: hipEvent_t the
 * dispatch itself stamps at its start and end (hipExtLaunchKernelGGL), or null for a plain launch. */
int exl3c4_dev_front(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_gemv(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_epilogue(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_dn(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1);
int exl3c4_dev_dequant(const void* record, int32_t rows, int32_t cols, int32_t bits, int32_t codebook, void* w_hat,
                       int64_t w_pitch, void* stream);

#ifdef __cplusplus
}
#endif

#endif
