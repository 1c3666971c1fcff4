/* exl3_oracle.h -- TEST INFRASTRUCTURE ONLY: the CPU restatement of the reference's EXL3 routed-expert path
 * that every device result of this repository is checked against.
 *
 * Nothing on the product path (the HIP library under radiance-exl3_amd/) links, loads or calls this code. Only
 * tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use it, and only as the checker or as the
 * timed CPU baseline.
 *
 * Scalar C99, built with -ffp-contract=off so that a product and a sum are two f32 roundings, as the reference's
 * host library computes them. Every function names the reference file:line whose semantics it restates:
 *   common/exl3_decode.c      fp16, codebooks, the tile map, tile streams and states, trellis decode, the codes
 *                             plane, the Hadamard-128, W_hat and W of one weight
 *   common/exl3_layout.c      canonical codes plane <-> exllamav3 tile-stream record
 *   kernels/exl3ref/ref.c     the op arithmetic (prep_gu, gate_up, down, gate_up_down), rounding points, zero rules
 *   include/exl3_abi.h        the routing contract (stable scatter) and the expert classes
 *   tests/ref/exl3_numpy.py   moe_scatter semantics (read as text)
 *
 * Parity pins (what checks each function against something it did not write) are listed in tests/test_oracle.py;
 * the op-level functions are pinned to tolerance by a float64 dense product and to the bit by invariants. */
#ifndef EXL3_ORACLE_H
#define EXL3_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum { OR_CB_3INST = 0, OR_CB_MCG = 1, OR_CB_MUL1 = 2 };
enum { OR_OK = 0, OR_E_ARG = -1, OR_E_SHAPE = -2, OR_E_NOMEM = -3 };

/* ---- fp16 / bf16 (common/exl3_decode.c:16-39; rad_f32_to_f16 / rad_f32_to_bf16 are plain RNE) */
float    or_half_to_float(uint16_t h);
uint16_t or_half_from_double(double x);
uint16_t or_f32_to_f16(float f);
uint16_t or_f32_to_bf16(float f);
float    or_bf16_to_f32(uint16_t b);
void     or_narrow(const float* in, uint16_t* bf16_out, uint16_t* f16_out, int64_t n);

/* ---- codebook (common/exl3_decode.c:43-67) */
uint16_t or_codebook_value(uint32_t state, int codebook);
/* All 65,536 states of one codebook, as fp16 bits. */
void     or_codebook_table(int codebook, uint16_t* out65536);

/* ---- the tile (common/exl3_decode.c:71-121) */
void or_pos_to_tile(int p, int* r, int* c);
int  or_tile_to_pos(int r, int c);
void or_tile_symbols(const uint16_t* tile, int bits, uint8_t* sym256);
void or_tile_pack(const uint8_t* sym256, int bits, uint16_t* tile);
void or_tile_states(const uint8_t* sym256, int bits, uint16_t* state256);
int  or_trellis_decode(const uint16_t* trellis, int64_t kt, int64_t nt, int bits, int codebook,
                       uint16_t* w_hat);

/* ---- the canonical codes plane (common/exl3_decode.c:148-168) and the record (common/exl3_layout.c:62-104) */
int64_t  or_codes_row_bytes(int64_t cols, int bits);
uint32_t or_codes_get(const uint8_t* codes, int64_t row_bytes, int bits, int64_t i, int64_t j);
void     or_codes_set(uint8_t* codes, int64_t row_bytes, int bits, int64_t i, int64_t j, uint32_t v);
int64_t  or_record_elems(int64_t rows, int64_t cols, int bits);
int      or_codes_to_record(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int bits,
                            uint16_t* record);
int      or_record_to_codes(const uint16_t* record, int64_t rows, int64_t cols, int bits, uint8_t* codes,
                            int64_t row_bytes);

/* ---- the rotation (common/exl3_decode.c:172-189) */
int or_had128(float* v, int64_t n);

/* ---- one weight (common/exl3_decode.c:193-271). codes: the canonical plane, rows row_bytes apart
 * (0 = dense). W_hat rows [row0, row0+n) as f32 [n][cols] (exact fp16 values); W rows likewise with both
 * rotations and scales in exllamav3's order (suh1: the up half's input scales of a stacked weight, or null). */
int or_decode_what_rows(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int bits,
                        int codebook, int64_t row0, int64_t n, float* out);
/* The same W_hat as fp16 bits [n][cols]: what the device dequant kernel is compared with, bit for bit. */
int or_decode_what_rows_f16(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int bits,
                            int codebook, int64_t row0, int64_t n, uint16_t* out);
int or_decode_rows(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int bits, int codebook,
                   const uint16_t* suh, const uint16_t* suh1, const uint16_t* svh, int64_t row0, int64_t n,
                   float* out);

/* ---- the ops (kernels/exl3ref/ref.c, docs/OPS-exl3.md "What they compute").
 *
 * One class of experts is a set of STACKED tables: entry j of plane p at base + j * stride (bytes). Class c
 * of an n_class op holds experts e with e % n_class == c at entry e / n_class (include/exl3_abi.h:847-853). */
typedef struct OrClass {
    int64_t        rows, cols;          /* this class's weight [N, K] (gate_up: N = 2W, gate rows then up rows) */
    const uint8_t* codes;  int64_t codes_stride;    /* canonical uK planes, dense rows */
    const uint16_t* suh;   int64_t suh_stride;      /* f16 [cols] */
    const uint16_t* suh1;  int64_t suh1_stride;     /* f16 [cols], gate_up / prep_gu only */
    const uint16_t* svh;   int64_t svh_stride;      /* f16 [rows] */
    const uint16_t* dn_suh; int64_t dn_suh_stride;  /* f16 [rows/2], gate_up h_rot = 1 only */
} OrClass;

typedef struct OrOp {
    int            op;          /* 0 down, 1 gate_up, 2 prep_gu (include/exl3_abi.h:292 numbering) */
    int            bits, codebook, n_class, h_rot, a_rot;
    int64_t        n_expert, top_k;
    OrClass        cls[4];
    const void*    x;           /* the input: token rows (gate_up a_rot 0, prep_gu), xr or h (sorted rows) */
    int            x_bf16;      /* 1: x is bf16 (token rows only) */
    int64_t        x_rows, x_pitch;                  /* elements */
    const int32_t* sorted_tok;
    const int32_t* expert_offset;                    /* [n_expert + 1] */
    void*          y;           /* gate_up h f16, down y bf16, prep_gu xr f16 */
    int64_t        T, y_pitch;
} OrOp;

/* Threads or_launch / or_gate_up_down spread the live experts over (OpenMP; default 1, the reference's serial loop).
 * The outputs do not depend on it: each expert's rows are computed by one thread in the serial order. */
void or_set_threads(int n);
int  or_get_threads(void);

/* Runs one op as kernels/exl3ref/ref.c:278-331 does (after its refusals: this entry assumes operands already
 * checked). Returns OR_OK, or OR_E_SHAPE / OR_E_NOMEM. */
int or_launch(const OrOp* o);

/* kernels/exl3ref/ref.c:27-32: xr = f16(had(f16(x * s))) over n values (x f32, s f16 bits), as f32. */
int or_prologue(const float* x, const uint16_t* s, int64_t n, float* xr);

/* gate_up(a_rot 0, h_rot 1) then down(h_rot 1): the gate_up_down definition (kernels/exl3ref/ref.c:235-276).
 * `gu` is the gate_up op (its y unused), `dn` the down op (its x unused); h is allocated here. */
int or_gate_up_down(const OrOp* gu, const OrOp* dn);

/* ---- routing (include/exl3_abi.h:90-158; tests/ref/exl3_numpy.py:223-242 read as text).
 * Stable counting sort of the flat (token, slot) index by expert; ids outside [expert_base, expert_base + n_expert)
 * are dropped. sorted_tok[n_tok*top_k] (-1 past the live count), expert_offset[n_expert + 1]. */
void or_moe_scatter(const int32_t* expert_ids, int64_t n_tok, int64_t top_k, int64_t expert_base,
                    int64_t n_expert, int32_t* sorted_tok, int32_t* expert_offset);
/* The same, with expert_count[n_expert] (rows per expert) and row_of[n_tok*top_k] (the sorted row of each flat pair,
 * -1 for a dropped pair); either may be null. */
void or_moe_scatter_full(const int32_t* expert_ids, int64_t n_tok, int64_t top_k, int64_t expert_base,
                         int64_t n_expert, int32_t* sorted_tok, int32_t* expert_offset, int32_t* expert_count,
                         int32_t* row_of);

/* router_topk (include/exl3_abi.h:96-98: softmax over ALL logits, top_k, optional renormalisation), in double: the
 * top_k ids ranked by probability with ties to the lower id (the softmax is monotone in the logit, so by logit; a NaN
 * logit ranks last), p_e = exp(l_e - m) / sum over all e of exp(l - m), renormalised over the top_k when asked;
 * expert_w as f32 of the double. */
void or_router_topk(const float* logits, int64_t n_tok, int64_t n_expert, int64_t pitch, int top_k, int renorm,
                    int32_t* expert_ids, float* expert_w);

/* moe_gather (include/exl3_abi.h:104-108, the north star's layer output): out[t][c] = f16 RNE of the f32 sum, over the
 * slots in ascending order with a row, of the f32 product expert_w[t][s] * y[row][c] (one rounding each). y bf16 or
 * f16 bits. */
void or_moe_gather(const uint16_t* y, int y_bf16, int64_t y_pitch, const float* expert_w, const int32_t* row_of,
                   int64_t n_tok, int top_k, int64_t cols, uint16_t* out, int64_t out_pitch);

#ifdef __cplusplus
}
#endif

#endif
