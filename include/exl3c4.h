/* exl3c4.h -- the C-ABI of exl3c4, an MI355X (gfx950, CDNA4, wave64) kernel library for radiance-exl3's routed-expert
 * hot path: the EXL3 trellis-coded mixture-of-experts ops moe_exl3_prep_gu, moe_exl3_gate_up, moe_exl3_down and
 * moe_exl3_gate_up_down.
 *
 * Two layers are exported from libexl3c4.so, both plain C (no torch or HIP types in any signature; a stream is an
 * opaque hipStream_t passed as void*):
 *
 *  1. THE OP ENTRY POINTS BELOW (exl3c4_*). Each replaces one entry of the reference device library's internal C-ABI
 *     (kernels/exl3r4d/exl3r4d_dev.h:75-109: exl3r4d_launch_gemm, exl3r4d_launch_prep, the fused gate_up_down launch)
 *     and carries the reference op contract (docs/OPS-exl3.md:84-191, include/exl3_abi.h:160-288) on plain pointers:
 *     what the radiance engine would hand over in RadArgs (kernels/exl3r4d/launch.c:150-250) arrives here already
 *     unpacked. Launches allocate nothing, synchronise nothing and read no environment (kernels/exl3r4d/launch.c:1-3);
 *     scratch is the caller's, sized by exl3c4_scratch_bytes from the geometry alone.
 *
 *  2. THE RADIANCE KERNEL-PLUGIN EXPORTS (rad_plugin_abi_version, rad_plugin_info, rad_kernel_schema_count/_at,
 *     rad_kernel_count/_at, rad_kernel_concurrent; include/rad_shim.h, radiance-exl3_amd/csrc/exl3c4_plugin.c), the
 *     same symbols the gfx1201 library exports (kernels/exl3r4d/rows.c:527-550), whose rows' launch hooks unpack RadArgs
 *     into the structs below.
 *
 * Return codes are radiance's (tests/ref/test_exl3ref.py:44, docs/STEP0.md row 1.72): 0 OK, negative refusals, always
 * returned BEFORE anything is written.
 *
 * THE STORED FORM of a codes plane (exl3c4_relayout). The canonical plane (include/exl3_encoding.h:12-13: uK, element
 * (i, j) = the K-bit symbol of W_hat[k = j][n = i], LSB-first rows) is re-laid once at load time into this library's
 * wave64 record: for a weight [N rows, K cols], blocks (strip nb = 0..N/32-1, kstep ks = 0..K/64-1) in nb-major order,
 * each block 64 segments of K u32 words, segment X (X = c + 16 g, c = 2 s + t) being stream words [sK, sK + K) of tile
 * (tk = 4 ks + g, tn = 2 nb + t) -- exactly the words one lane of a wave decodes for one 16x16x32 MFMA step. A lossless
 * permutation of the exllamav3 tile stream (common/exl3_layout.c:62-104); exl3c4_unrelayout inverts it.
 */
#ifndef EXL3C4_H
#define EXL3C4_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define EXL3C4_ABI_VERSION 1

/* radiance status codes (names at kernels/exl3r4d/launch.c:5-14; values tests/ref/test_exl3ref.py:44). */
enum {
    EXL3C4_OK = 0,
    EXL3C4_E_SHAPE = -1,
    EXL3C4_E_DTYPE = -2,
    EXL3C4_E_ALIGN = -3,
    EXL3C4_E_STRIDE = -4,
    EXL3C4_E_SCHEMA = -9,
    EXL3C4_E_INVAL = -12,
    EXL3C4_E_UNSUPPORTED = -18,
    EXL3C4_E_SCRATCH = -20,
    EXL3C4_E_DEVICE = -21,
    /* the import's (quantizers/exl3/exl3_quant.cpp:12-20 names them; radiance's values are not in the reference, these
     * are this library's; FORMAT is include/rad_shim.h's) */
    EXL3C4_E_FORMAT = -5,
    EXL3C4_E_NOTFOUND = -30,
    EXL3C4_E_IO = -31,
};

/* The ops, numbered as include/exl3_abi.h:292 numbers them. */
enum { EXL3C4_DOWN = 0, EXL3C4_GATE_UP = 1, EXL3C4_PREP_GU = 2, EXL3C4_GU_DN = 3 };
/* Codebooks, numbered as common/exl3_decode.h:60 numbers them. */
enum { EXL3C4_CB_3INST = 0, EXL3C4_CB_MCG = 1, EXL3C4_CB_MUL1 = 2 };
/* Activation dtypes. */
enum { EXL3C4_F16 = 0, EXL3C4_BF16 = 1, EXL3C4_F32 = 2 };

/* One class of experts (include/exl3_abi.h:186-206, 298-304): a weight table per plane. A table is a device pointer
 * array (its *_stride 0: entry j at ((void**)base)[j], the engine's form) or one stacked device buffer (entry j at base
 * + j * stride bytes, a tool's form). Class c of an n_class op holds experts e % n_class == c at entry e / n_class.
 *   codes   the STORED record (exl3c4_relayout) of the expert's [rows, cols] weight
 *   suh     f16 [cols]; suh1 f16 [cols] (gate_up / prep_gu: the up half's input scales)
 *   svh     f16 [rows]; dn_suh f16 [rows / 2] (gate_up h_rot = 1: DOWN's suh of the same expert) */
typedef struct Exl3c4Class {
    int32_t     rows, cols;
    const void* codes;
    const void* suh;
    const void* suh1;
    const void* svh;
    const void* dn_suh;
    int64_t     codes_stride, suh_stride, suh1_stride, svh_stride, dn_suh_stride;
} Exl3c4Class;

/* One launch of one op (docs/OPS-exl3.md "The ops"). Every pointer is device memory.
 *   x        gate_up a_rot 0 / prep_gu / gate_up_down: token rows [x_rows, >= max cols], f16 or bf16;
 *            gate_up a_rot 1: prep_gu's xr [T, >= 2 max cols] f16; down: h [T, >= max cols] f16
 *   y        gate_up: h f16 [T, max rows / 2]; down / gate_up_down: y bf16 [T, max rows]; prep_gu: xr f16
 *            [T, 2 max cols] (rows outside the runs and columns past 2 C left as they were)
 *   gate_up_down: cls[] is gate_up's geometry (with dn_suh), dn[] down's codes and svh ([cols, rows / 2] a class). */
typedef struct Exl3c4Op {
    int32_t        op;
    int32_t        bits, codebook;
    int32_t        n_class;            /* 1, 2 (the two-class ops) or 4 (the _mod4 forms) */
    int32_t        h_rot, a_rot;
    int64_t        M, n_expert, top_k; /* M: the band's token count, sizes scratch (include/exl3_abi.h:155-157) */
    Exl3c4Class    cls[4];
    Exl3c4Class    dn[4];
    const void*    x;
    int32_t        x_dtype;
    int64_t        x_rows, x_cols, x_pitch;   /* elements */
    const int32_t* sorted_tok;                /* [>= T] */
    const int32_t* expert_offset;             /* [n_expert + 1] */
    void*          y;
    int64_t        T, y_cols, y_pitch;        /* rows, width, pitch (elements) of the output */
    int32_t        dn_bits;                   /* gate_up_down: down's K when it differs from gate_up's (bits);
                                                 0 = bits. No counterpart in the reference's op, which takes one K:
                                                 a layer of mixed K runs there as gate_up then down */
} Exl3c4Op;

/* Bytes of scratch a launch of this op needs, from its parameters only (M * top_k rows at the band top, the classes'
 * geometry): docs/STEP0.md:142-146, kernels/exl3r4d/launch.c:263-275. Negative: the refusal the launch would give. */
int64_t exl3c4_scratch_bytes(const Exl3c4Op* op);

/* The bytes of scratch THIS launch of `op` (its T sorted rows) needs: exl3c4_launch refuses EXL3C4_E_SCRATCH below it.
 * Never more than exl3c4_scratch_bytes(op), which is the largest of these over every row count up to the band top, so
 * scratch sized once for the band takes every smaller batch. A query with no counterpart in the reference. */
int64_t exl3c4_launch_scratch_bytes(const Exl3c4Op* op);

/* The same from the geometry alone (no operands): the op, its classes' [rows, cols] as the op's weights are (for
 * gate_up_down: gate_up's), M tokens (a band's top), top_k and n_expert. What a plugin's scratch hook answers from
 * the parameters (docs/STEP0.md:142-146). A negative status for a geometry the op refuses. */
int64_t exl3c4_scratch_bytes_geom(int32_t op, int32_t n_class, const int32_t* rows, const int32_t* cols, int64_t M,
                                  int64_t top_k, int64_t n_expert);

/* Checks, then launches, one op on `stream` (kernels/exl3r4d/launch.c:525-612, 687-790, 833-855). Nothing is written
 * before every refusal has been decided. `scratch` is device memory of at least exl3c4_scratch_bytes, 256-B aligned. */
int exl3c4_launch(const Exl3c4Op* op, void* scratch, int64_t scratch_bytes, void* stream);

/* gate_up_down's single kernel (the decode path from EXL3C4_GD_FUSE_MIN_T sorted rows) orders its workgroups through
 * a block of counters -- a status word and two counters a sorted row (and a line a token for exl3c4_launch_gather) -- that must be zero when it starts and that it
 * leaves zero again when it ends well (each row's last down unit zeroes the row's). exl3c4_launch zeroes them in its
 * scratch before every launch (one more dispatch). exl3c4_launch_ctr takes them from `ctr` instead: a device block of
 * at least exl3c4_ctr_bytes, 256-B aligned, that the caller zeroed once (hipMemset) and keeps -- the reference's
 * counter pool, which its row instance's init allocates and zeroes and whose blocks the fused launch leaves zero
 * (kernels/exl3r4d/launch.c:311-324; the fused launch's `ctr` argument, launch.c:464-466). The block's first int32 is
 * the status word exl3c4_scratch_status describes (0: good); after a launch that left it nonzero, zero the block again.
 * Two launches that may overlap (two streams) need two blocks; launches that share one are ordered on one stream. A
 * launch that does not run that kernel does not read ctr: exl3c4_launch_ctr is then exl3c4_launch. */
int64_t exl3c4_ctr_bytes(const Exl3c4Op* op);
int exl3c4_launch_ctr(const Exl3c4Op* op, void* scratch, int64_t scratch_bytes, void* stream, void* ctr,
                      int64_t ctr_bytes);

/* exl3c4_launch_ctr, then moe_gather of its output: exactly exl3c4_launch_ctr(op, ...) followed by
 * exl3c4_moe_gather(op->y, EXL3C4_BF16, op->y_pitch, expert_w, row_of, op->M, op->top_k, op->y_cols, out, out_pitch)
 * -- the same bits in y and out, and the same refusals. When gate_up_down runs as its single kernel and `ctr` is given
 * (exl3c4_ctr_bytes covers a counter line a token after the rows'), the gather rides in that kernel: the down unit that
 * completes a token's rows of a 128-column block sums that block, so the layer's step has no gather dispatch and no
 * gather startup after the last down unit. Otherwise the two run one after the other. row_of must be the inverse of
 * op->sorted_tok (what the scatter writes). op: gate_up_down or down. The reference's engine dispatches the two
 * separately (include/exl3_abi.h:90-158); no counterpart there. */
int exl3c4_launch_gather(const Exl3c4Op* op, void* scratch, int64_t scratch_bytes, void* stream, void* ctr,
                         int64_t ctr_bytes, const float* expert_w, const int32_t* row_of, void* out,
                         int64_t out_pitch);

/* THE LAUNCH THAT ALLOCATES NOTHING. No counterpart in the reference: for callers that cannot allocate or pass a
 * workspace -- code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc. exl3c4_launch_noalloc
 * is exl3c4_launch (the same kernels, the same bits) with the library's own scratch: a file-scope device array of
 * EXL3C4_NOALLOC_SCRATCH_BYTES, one on each GPU the library runs on, held until the process ends; the launch itself
 * allocates nothing. A launch whose scratch (exl3c4_launch_scratch_bytes) exceeds it is refused with EXL3C4_E_SCRATCH
 * before anything is written (at the configs' geometry -- gate/up 2048 -> 512, 512 experts -- that covers the decode
 * band to M = 64 tokens of top-10 and small prefills). `stream` must belong to the current device (else
 * EXL3C4_E_DEVICE). Every call on one GPU shares that GPU's array and leaves its contents behind: calls that may
 * overlap on one GPU (two streams, two threads) race and must be ordered by the caller. */
#define EXL3C4_NOALLOC_SCRATCH_BYTES (16ll << 20)
int64_t exl3c4_noalloc_scratch_bytes(void);
int     exl3c4_launch_noalloc(const Exl3c4Op* op, void* stream);

/* The kernels a launch can run: prep_gu's rotation; gate_up's GEMM (with its input rotation), then for gate_up alone
 * its epilogue; down's GEMM with its epilogue (in gate_up_down it also forms h from gate_up's partial sums); and
 * gate_up_down's single kernel, which runs both GEMMs in one dispatch at decode once T >= EXL3C4_GD_FUSE_MIN_T.
 * exl3c4_launch_timed refuses (EXL3C4_E_INVAL) a kernel that the launch does not run. */
enum { EXL3C4_K_PREP = 0, EXL3C4_K_GATE_UP = 1, EXL3C4_K_EPI_GU = 2, EXL3C4_K_DOWN = 3, EXL3C4_K_GATE_UP_DOWN = 4 };
#define EXL3C4_GD_FUSE_MIN_T 32

/* The least sorted-row count T at which gate_up, down and gate_up_down over n_expert experts take the prefill path (a
 * chunk plan and one GEMM kernel a projection, decoding each weight once a chunk of up to 112 rows of one expert, 96
 * where the launch's K exceed 4) rather than the decode kernels: max(64, ceil(7 n_expert / 8)) -- the crossover
 * measured on MI355X at the decode layer's experts. A function of T and n_expert only, never of the routing. A query
 * with no counterpart in the reference (whose rows split the band at M = 17, kernels/exl3r4d/rows.c:255-315). */
int64_t exl3c4_prefill_min_rows(int64_t n_expert);

/* exl3c4_launch, with kernel `kernel` of the sequence dispatched so that the dispatch itself stamps ev_start and
 * ev_stop (two hipEvent_t the caller created) at its start and end: the duration of that one kernel, read with
 * hipEventElapsedTime, however the host paces the launches. A measurement entry with no counterpart in the reference
 * (whose device library times kernels with compile-time timestamp arms, kernels/exl3r4d/exl3r4d.hip:135-136); the bits
 * written are exl3c4_launch's. */
int exl3c4_launch_timed(const Exl3c4Op* op, void* scratch, int64_t scratch_bytes, void* stream, int32_t kernel,
                        void* ev_start, void* ev_stop);

/* exl3c4_launch, and on the prefill path (a chunk plan: from exl3c4_prefill_min_rows sorted rows) its GEMMs also write
 * their f32 accumulations to scratch for exl3c4_scratch_partials -- 4 bytes a row and output column each, which the
 * production launch does not spend. The outputs are exl3c4_launch's, bit for bit. A checker's entry; no counterpart
 * in the reference. */
int exl3c4_launch_checked(const Exl3c4Op* op, void* scratch, int64_t scratch_bytes, void* stream);

/* Where a launch of `op` leaves the f32 accumulations of its GEMM (gemm 0: gate_up's, or down's for the down op; 1:
 * gate_up_down's down) in its scratch: acc[row][col] = sum over s < *splits of the f32 at scratch + *offset +
 * 4 * (s * *split_stride + row * *pitch + col), for the live rows. The epilogue adds them in this order. Every
 * decode-path launch leaves them; a prefill-path launch only through exl3c4_launch_checked. For a checker of the
 * accumulation itself (the values before any narrowing); no counterpart in the reference. */
int exl3c4_scratch_partials(const Exl3c4Op* op, int32_t gemm, int64_t* offset, int64_t* pitch, int64_t* split_stride,
                            int32_t* splits);

/* Where a launch of `op` that runs gate_up_down's single kernel leaves its status word in its scratch (an int32 at
 * scratch + *offset): 0 after a good launch; 1 when a down unit's wait for its row's gate_up units gave up (after
 * 0.5 s), and the output is then void. EXL3C4_E_INVAL when the launch does not run that kernel. A checker's entry;
 * no counterpart in the reference. */
int exl3c4_scratch_status(const Exl3c4Op* op, int64_t* offset);

/* W_hat of one stored weight [rows, cols] as fp16 bits [rows][w_pitch] on the device -- the same decode the GEMMs run,
 * exposed so it can be compared bit for bit with common/exl3_decode.c:193-221. bits 1..8 (K = 1 is decoder-only,
 * include/exl3_encoding.h:45-48). */
int exl3c4_dequant(const void* record, int32_t rows, int32_t cols, int32_t bits, int32_t codebook, void* w_hat,
                   int64_t w_pitch, void* stream);

/* ------------------------------------------------------------------ the routing around the ops (device)
 * What the radiance engine runs in front of and behind the routed-expert ops (router_topk, moe_scatter, moe_gather;
 * the contract at include/exl3_abi.h:90-158), so that a whole MoE layer runs on this library. No counterpart in the
 * reference device library, which leaves them to the engine; the semantics are the contract's and
 * tests/ref/exl3_numpy.py:223-242's (the scatter). Each returns before writing anything when it refuses. */

/* The router: for each of n_tok tokens, the softmax over all n_expert logits (row t at logits + t * pitch elements,
 * dtype EXL3C4_F32 / F16 / BF16), its top_k experts by probability -- ties to the lower id; the softmax is monotone in
 * the logit, so they are ranked by logit -- and their probabilities, renormalised to sum to one when renorm is 1:
 * expert_ids i32 [n_tok][top_k] (descending probability), expert_w f32 [n_tok][top_k]. f32 arithmetic: m = max logit,
 * p_e = expf(l_e - m) / sum over all e. 1 <= top_k <= min(n_expert, 64), n_expert <= 1024. */
int exl3c4_router_topk(const void* logits, int32_t logits_dtype, int64_t n_tok, int64_t n_expert, int64_t pitch,
                       int32_t top_k, int32_t renorm, int32_t* expert_ids, float* expert_w, void* stream);

/* moe_scatter: the flat pairs p = t * top_k + slot (T = n_tok * top_k of them) grouped by expert by a STABLE counting
 * sort (include/exl3_abi.h:109-123): expert_offset i32 [n_expert + 1] (expert e's rows [off[e], off[e+1]), off[n_expert]
 * the live count), sorted_tok i32 [T] (-1 past the live count), and, when not null, expert_count i32 [n_expert] and
 * row_of i32 [T] (the sorted row of pair p, -1 for a dropped pair: what the gather reads). A pair whose expert is
 * outside [expert_base, expert_base + n_expert) is dropped. One workgroup; n_expert <= 2048. */
int exl3c4_moe_scatter(const int32_t* expert_ids, int64_t n_tok, int32_t top_k, int64_t expert_base,
                       int64_t n_expert, int32_t* sorted_tok, int32_t* expert_offset, int32_t* expert_count,
                       int32_t* row_of, void* stream);

/* router_topk_scatter: the two above on the same logits (the fused form the contract names, include/exl3_abi.h:96-98),
 * with expert_base 0; up to 16 tokens in one workgroup (one launch), more as the two launches. */
int exl3c4_router_topk_scatter(const void* logits, int32_t logits_dtype, int64_t n_tok, int64_t n_expert,
                               int64_t pitch, int32_t top_k, int32_t renorm, int32_t* expert_ids, float* expert_w,
                               int32_t* sorted_tok, int32_t* expert_offset, int32_t* expert_count, int32_t* row_of,
                               void* stream);

/* moe_gather: out[t][c] = f16( sum over slots s = 0 .. top_k-1 in ascending order, of the pairs with a row, of
 * expert_w[t][s] * y[row_of[t * top_k + s]][c] ), accumulated in f32 as one product and one add a slot (the north
 * star's layer output: the weighted sum in fp32, cast to fp16, round to nearest even). y: the down op's output rows,
 * dtype EXL3C4_BF16 or F16, y_pitch elements apart; out f16, out_pitch apart. cols % 8 == 0. */
int exl3c4_moe_gather(const void* y, int32_t y_dtype, int64_t y_pitch, const float* expert_w, const int32_t* row_of,
                      int64_t n_tok, int32_t top_k, int64_t cols, void* out, int64_t out_pitch, void* stream);

/* ------------------------------------------------------------------ the stored form (host, load time) */
/* Bytes of the stored record of a [rows, cols] weight at K bits: rows * cols * K / 8. */
int64_t exl3c4_record_bytes(int64_t rows, int64_t cols, int32_t bits);
/* Canonical uK plane (rows row_bytes apart; 0 = dense) -> stored record (kernels/exl3r4d/layout.c:269-330 is the
 * reference's hook for the same step). rows % 32 == 0 and cols % 64 == 0, bits 1..8. */
int exl3c4_relayout(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int32_t bits, void* record);
/* Stored record -> canonical plane (kernels/exl3r4d/layout.c:332-360): the bits of each row's elements are written,
 * the rest of the plane is left as it was. */
int exl3c4_unrelayout(const void* record, int64_t rows, int64_t cols, int32_t bits, uint8_t* codes, int64_t row_bytes);
/* exllamav3's tile record of a [rows, cols] weight (int16 [cols / 16][rows / 16][16 K], a checkpoint's .trellis) ->
 * canonical plane (common/exl3_layout.c:38-56, exl3_record_to_codes). rows, cols in 16s, bits 1..8; row_bytes 0 =
 * dense. */
int exl3c4_record_to_codes(const uint16_t* record, int64_t rows, int64_t cols, int32_t bits, uint8_t* codes,
                           int64_t row_bytes);

/* ------------------------------------------------------------------ the import (host, load time)
 * Routed experts of an EXL3 checkpoint directory (exllamav3's safetensors layout: config.json with
 * quantization_config.quant_method "exl3", model.safetensors or shards named by model.safetensors.index.json) into
 * canonical planes: what the reference's `exl3` quantiser does (quantizers/exl3/exl3_quant.cpp:192-256; its reader
 * quantizers/exl3/exl3_src.cpp). A checkpoint is opened once and may be shared by threads.
 *   exl3c4_ckpt_open          EXL3C4_E_FORMAT: not an EXL3 checkpoint this reader understands (no config.json, another
 *                             quant_method, no layer count, a malformed header or index); EXL3C4_E_IO
 *   exl3c4_ckpt_layers        text_config.num_hidden_layers (or num_hidden_layers): layer index of the MTP head
 *   exl3c4_import_parse_name  blk.L.ffn_gate_up_exps.E.weight (stacked 1) | blk.L.ffn_down_exps.E.weight (stacked 0);
 *                             anything else EXL3C4_E_UNSUPPORTED (exl3_quant.cpp:97-114)
 *   exl3c4_import_weight      the named weight [rows, cols] (stacked: gate rows then up rows) into codes (uK, rows
 *                             row_bytes apart), suh [cols], suh1 [cols] (stacked only: the up half's), svh [rows].
 *                             Refusals (exl3_quant.cpp:12-20, 142-247), before any plane is written:
 *                               UNSUPPORTED  not a routed-expert name; a .bias; half-integer K (last dim 16 K + 8)
 *                               INVAL        bits outside 2..8, an unknown codebook, a plane missing
 *                               SHAPE        rows / cols not in 128s (a stacked weight's halves too); a trellis whose
 *                                            tiles are another [cols, rows]; suh / svh of another dtype or length
 *                               NOTFOUND     a layer past the layers and the MTP head; a missing trellis, suh or svh
 *                               DTYPE        a trellis of another K; a marker naming another codebook
 *                               FORMAT       a trellis not I16 rank 3 or its last dim not in 16s; a marker not an I32
 *                                            scalar, holding a wrong value, or both markers present
 *                               IO           a read that failed */
typedef struct Exl3c4Ckpt Exl3c4Ckpt;
int     exl3c4_ckpt_open(const char* dir, Exl3c4Ckpt** out);
void    exl3c4_ckpt_close(Exl3c4Ckpt* ckpt);
int64_t exl3c4_ckpt_layers(const Exl3c4Ckpt* ckpt);
int     exl3c4_import_parse_name(const char* name, int32_t* layer, int64_t* expert, int32_t* stacked);
int     exl3c4_import_weight(Exl3c4Ckpt* ckpt, const char* name, int32_t bits, int32_t codebook, int64_t rows,
                             int64_t cols, uint8_t* codes, int64_t row_bytes, uint16_t* suh, uint16_t* suh1,
                             uint16_t* svh);

/* ------------------------------------------------------------------ the plugin rows' instances (checkers' entries)
 * The gate_up_down rows' init hooks return an instance holding a pool of counter blocks, one per (stream, output) pair,
 * each with a host-visible flag the single decode kernel sets when a bounded wait gives up; the next launch on that
 * block reports RAD_E_DEVICE. No counterpart in the reference's exports (its pool is internal): for tests and tools.
 *   exl3c4_plugin_inst_flag          block's flag; when set >= 0 it is then written (a test forcing the failure path)
 *   exl3c4_plugin_inst_blocks_used   the blocks handed out so far */
int32_t exl3c4_plugin_inst_flag(void* inst, int32_t block, int32_t set);
int32_t exl3c4_plugin_inst_blocks_used(void* inst);
/* The device address of an instance's counter block `block` (its status word first, then a counter a sorted row, 256
 * bytes apart) and its size in bytes, or null past the blocks handed out: for a test that drives the kernel's own
 * failure report from the host (a status word set before a launch, a counter no count can complete). */
void*   exl3c4_plugin_inst_block(void* inst, int32_t block, int64_t* bytes);

/* ------------------------------------------------------------------ the narrowing conversions (checkers' entries)
 * The device's own f32 -> bf16 and f32 -> f16 conversions, as the kernels' outputs use them (down's y: one
 * v_cvt_pk_bf16_f32 for two values; h: round to nearest even on an f32 value), over n f32 values: out[j] = the 16-bit
 * result of in[j]. For a checker that holds them to the reference's rules (rad_f32_to_bf16: round to nearest even, a
 * nan kept quiet as (u >> 16) | 0x40; rad_f32_to_f16: IEEE round to nearest even) over every input class. No
 * counterpart in the reference. Returns 0 or EXL3C4_E_DEVICE; EXL3C4_E_SHAPE for n < 0 or n > 2^40. */
int exl3c4_check_narrow(const float* in, uint16_t* out_bf16, uint16_t* out_f16, int64_t n, void* stream);

/* Library identity: "gfx950" and the ABI version above. */
const char* exl3c4_build_target(void);
int         exl3c4_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif
