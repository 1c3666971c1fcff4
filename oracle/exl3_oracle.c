/* exl3_oracle.c -- TEST INFRASTRUCTURE ONLY (see exl3_oracle.h): the CPU restatement the device library is
 * checked against. Scalar and slow on purpose; build with -ffp-contract=off. */
#include "exl3_oracle.h"

#include <math.h>
#include <stdlib.h>
#include <string.h>

/* =========================================================================================== fp16 / bf16 */

/* common/exl3_decode.c:16-23: a half is (1024 + m) * 2^(e - 25) for a normal exponent, m * 2^-24 below it. */
float or_half_to_float(uint16_t h) {
    const int e = (h >> 10) & 31, m = h & 1023;
    float mag;
    if (e == 31) mag = m ? NAN : INFINITY;
    else if (e == 0) mag = ldexpf((float)m, -24);
    else mag = ldexpf((float)(1024 + m), e - 25);
    return (h & 0x8000u) ? -mag : mag;
}

/* common/exl3_decode.c:25-39: one round-to-nearest-even of the exact double, inf at or past 65520, nan 0x7E00. */
uint16_t or_half_from_double(double x) {
    const uint16_t s = signbit(x) ? 0x8000u : 0u;
    double a = fabs(x), frac;
    int e;
    if (isnan(x)) return 0x7E00u;
    if (a >= 65520.0) return (uint16_t)(s | 0x7C00u);
    if (a < ldexp(1.0, -14)) return (uint16_t)(s | (uint16_t)nearbyint(a * ldexp(1.0, 24)));
    frac = frexp(a, &e);                       /* a = frac * 2^e, frac in [0.5, 1) */
    frac = nearbyint(ldexp(frac, 11));         /* 11 significant bits, RNE: [1024, 2048] */
    if (frac == 2048.0) { frac = 1024.0; ++e; }
    if (e + 14 >= 31) return (uint16_t)(s | 0x7C00u);
    return (uint16_t)(s | (uint16_t)((e + 14) << 10) | (uint16_t)(frac - 1024.0));
}

/* radiance's rad_f32_to_f16: the f32 value (exact in double) rounded once. */
uint16_t or_f32_to_f16(float f) { return or_half_from_double((double)f); }

/* radiance's rad_f32_to_bf16: round to nearest even on the f32 bits; nan stays a quiet nan. */
uint16_t or_f32_to_bf16(float f) {
    uint32_t u;
    memcpy(&u, &f, 4);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x0040u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

/* or_f32_to_bf16 and or_f32_to_f16 over an array (a checker's vector form of the two above). */
void or_narrow(const float* in, uint16_t* bf, uint16_t* h, int64_t n) {
    for (int64_t j = 0; j < n; ++j) {
        bf[j] = or_f32_to_bf16(in[j]);
        h[j] = or_f32_to_f16(in[j]);
    }
}

float or_bf16_to_f32(uint16_t b) {
    const uint32_t u = (uint32_t)b << 16;
    float f;
    memcpy(&f, &u, 4);
    return f;
}

/* =========================================================================================== codebook */

/* common/exl3_decode.c:43-67. mul1: fp16(1024 + bytesum(x * 0x83DCD12D)) * K_INV + K_BIAS, one fp16 rounding
 * (the product and sum are exact in double). mcg / 3inst: a 32-bit hash, (h & 0x8FFF8FFF) ^ 0x3B603B60, then the
 * two fp16 halves added with one rounding. */
#define OR_MUL1_MULT 0x83DCD12Du
#define OR_MCG_MULT  0xCBAC1FEDu
#define OR_MUL1_KINV 0x1EEEu
#define OR_MUL1_KBIAS 0xC931u

uint16_t or_codebook_value(uint32_t state, int codebook) {
    uint32_t x = state & 0xFFFFu;
    switch (codebook) {
    case OR_CB_MUL1: {
        const uint32_t h = x * OR_MUL1_MULT;
        const uint32_t sum = (h & 255u) + ((h >> 8) & 255u) + ((h >> 16) & 255u) + (h >> 24);
        const double kinv = (double)or_half_to_float(OR_MUL1_KINV), kbias = (double)or_half_to_float(OR_MUL1_KBIAS);
        return or_half_from_double((1024.0 + (double)sum) * kinv + kbias);
    }
    case OR_CB_MCG:   x = x * OR_MCG_MULT; break;
    case OR_CB_3INST: x = x * 89226354u + 64248484u; break;
    default:          return 0x7E00u;
    }
    x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
    return or_half_from_double((double)or_half_to_float((uint16_t)x) + (double)or_half_to_float((uint16_t)(x >> 16)));
}

void or_codebook_table(int codebook, uint16_t* out) {
    for (uint32_t s = 0; s < 65536u; ++s) out[s] = or_codebook_value(s, codebook);
}

/* =========================================================================================== the tile */

/* common/exl3_decode.c:71-82: position p = 8L + j sits at tile row (k axis) 2(L%4) + {0,1,8,9}[j%4] and tile
 * column (n axis) L/4 + 8(j/4). */
void or_pos_to_tile(int p, int* r, int* c) {
    const int L = p >> 3, j = p & 7;
    *r = 2 * (L & 3) + ((j & 1) | ((j & 2) << 2));
    *c = (L >> 2) + 8 * (j >> 2);
}

int or_tile_to_pos(int r, int c) {
    const int L = 4 * (c & 7) + ((r & 7) >> 1);
    const int j = 4 * (c >> 3) + (r & 1) + 2 * (r >> 3);
    return 8 * L + j;
}

/* Stream bit b of a tile (MSB first): bit 31 - b%32 of the little-endian u32 made of u16 [2w, 2w+1], w = b/32
 * (common/exl3_decode.c:84-88). */
static unsigned tile_bit(const uint16_t* tile, int b) {
    const int w = b >> 5;
    const uint32_t word = (uint32_t)tile[2 * w] | ((uint32_t)tile[2 * w + 1] << 16);
    return (word >> (31 - (b & 31))) & 1u;
}

/* common/exl3_decode.c:90-97 */
void or_tile_symbols(const uint16_t* tile, int bits, uint8_t* sym) {
    for (int p = 0; p < 256; ++p) {
        unsigned v = 0;
        for (int i = 0; i < bits; ++i) v = (v << 1) | tile_bit(tile, p * bits + i);
        sym[p] = (uint8_t)v;
    }
}

/* common/exl3_decode.c:99-109 */
void or_tile_pack(const uint8_t* sym, int bits, uint16_t* tile) {
    memset(tile, 0, (size_t)16 * (size_t)bits * sizeof(uint16_t));
    for (int p = 0; p < 256; ++p)
        for (int i = 0; i < bits; ++i) {
            if (!((sym[p] >> (bits - 1 - i)) & 1u)) continue;
            const int b = p * bits + i, w = b >> 5, sh = 31 - (b & 31);
            if (sh >= 16) tile[2 * w + 1] |= (uint16_t)(1u << (sh - 16));
            else tile[2 * w] |= (uint16_t)(1u << sh);
        }
}

/* common/exl3_decode.c:111-121: the 16-bit window ending at symbol p's last bit, circular within the tile. */
void or_tile_states(const uint8_t* sym, int bits, uint16_t* state) {
    const int reach = (16 + bits - 1) / bits;
    const uint32_t mask = (1u << bits) - 1u;
    for (int p = 0; p < 256; ++p) {
        uint32_t acc = 0;
        for (int q = p - reach + 1; q <= p; ++q) acc = (acc << bits) | (sym[(q + 256) & 255] & mask);
        state[p] = (uint16_t)acc;
    }
}

static int bits_ok(int bits) { return bits >= 1 && bits <= 8; }
static int cb_ok(int cb) { return cb == OR_CB_3INST || cb == OR_CB_MCG || cb == OR_CB_MUL1; }

/* common/exl3_decode.c:127-144: exllamav3's record int16 [kt][nt][16K] -> W_hat [16kt][16nt] ([k][n]). */
int or_trellis_decode(const uint16_t* trellis, int64_t kt, int64_t nt, int bits, int codebook, uint16_t* w_hat) {
    uint8_t sym[256];
    uint16_t st[256];
    if (!trellis || !w_hat || kt < 0 || nt < 0 || !bits_ok(bits) || !cb_ok(codebook)) return OR_E_ARG;
    for (int64_t tk = 0; tk < kt; ++tk)
        for (int64_t tn = 0; tn < nt; ++tn) {
            or_tile_symbols(trellis + (tk * nt + tn) * 16 * bits, bits, sym);
            or_tile_states(sym, bits, st);
            for (int p = 0; p < 256; ++p) {
                int r, c;
                or_pos_to_tile(p, &r, &c);
                w_hat[(tk * 16 + r) * (nt * 16) + tn * 16 + c] = or_codebook_value(st[p], codebook);
            }
        }
    return OR_OK;
}

/* =========================================================================================== the codes plane */

/* common/exl3_decode.c:148-168: element (i, j) of a uK plane is bits [jK, (j+1)K) of row i, LSB first. */
int64_t or_codes_row_bytes(int64_t cols, int bits) { return (cols * bits + 7) / 8; }

uint32_t or_codes_get(const uint8_t* codes, int64_t row_bytes, int bits, int64_t i, int64_t j) {
    const uint8_t* row = codes + i * row_bytes;
    uint32_t v = 0;
    for (int k = 0; k < bits; ++k) {
        const int64_t b = j * bits + k;
        v |= (uint32_t)((row[b >> 3] >> (b & 7)) & 1u) << k;
    }
    return v;
}

void or_codes_set(uint8_t* codes, int64_t row_bytes, int bits, int64_t i, int64_t j, uint32_t v) {
    uint8_t* row = codes + i * row_bytes;
    for (int k = 0; k < bits; ++k) {
        const int64_t b = j * bits + k;
        const uint8_t m = (uint8_t)(1u << (b & 7));
        if ((v >> k) & 1u) row[b >> 3] |= m;
        else row[b >> 3] &= (uint8_t)~m;
    }
}

/* common/exl3_layout.c:62-104: the record of a rows x cols rectangle is int16 [cols/16][rows/16][16K], tile (tk, tn)
 * holding W_hat[k = 16tk + r][n = 16tn + c] at position or_tile_to_pos(r, c), whose symbol the plane keeps at
 * element (n, k). */
int64_t or_record_elems(int64_t rows, int64_t cols, int bits) { return (rows / 16) * (cols / 16) * 16 * bits; }

int or_codes_to_record(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int bits,
                       uint16_t* record) {
    uint8_t sym[256];
    const int64_t nt = rows / 16, kt = cols / 16;
    if (!codes || !record || !bits_ok(bits)) return OR_E_ARG;
    if (rows < 0 || cols < 0 || rows % 16 || cols % 16 || row_bytes < or_codes_row_bytes(cols, bits))
        return OR_E_SHAPE;
    for (int64_t tk = 0; tk < kt; ++tk)
        for (int64_t tn = 0; tn < nt; ++tn) {
            for (int p = 0; p < 256; ++p) {
                int r, c;
                or_pos_to_tile(p, &r, &c);
                sym[p] = (uint8_t)or_codes_get(codes, row_bytes, bits, tn * 16 + c, tk * 16 + r);
            }
            or_tile_pack(sym, bits, record + (tk * nt + tn) * 16 * bits);
        }
    return OR_OK;
}

int or_record_to_codes(const uint16_t* record, int64_t rows, int64_t cols, int bits, uint8_t* codes,
                       int64_t row_bytes) {
    uint8_t sym[256];
    const int64_t nt = rows / 16, kt = cols / 16;
    if (!codes || !record || !bits_ok(bits)) return OR_E_ARG;
    if (rows < 0 || cols < 0 || rows % 16 || cols % 16 || row_bytes < or_codes_row_bytes(cols, bits))
        return OR_E_SHAPE;
    for (int64_t tk = 0; tk < kt; ++tk)
        for (int64_t tn = 0; tn < nt; ++tn) {
            or_tile_symbols(record + (tk * nt + tn) * 16 * bits, bits, sym);
            for (int p = 0; p < 256; ++p) {
                int r, c;
                or_pos_to_tile(p, &r, &c);
                or_codes_set(codes, row_bytes, bits, tn * 16 + c, tk * 16 + r, sym[p]);
            }
        }
    return OR_OK;
}

/* =========================================================================================== the rotation */

/* common/exl3_decode.c:172-189: per block of 128, butterfly stages h = 1, 2, .., 64 with (a + b) low and (a - b)
 * high, in f32, then one multiply by (float)(1/sqrt(128)). */
int or_had128(float* v, int64_t n) {
    const float scale = 0.08838834764831844055f;
    if (!v || n < 0 || n % 128) return OR_E_SHAPE;
    for (int64_t base = 0; base < n; base += 128) {
        float* x = v + base;
        for (int h = 1; h < 128; h *= 2)
            for (int i = 0; i < 128; i += 2 * h)
                for (int j = i; j < i + h; ++j) {
                    const float a = x[j], b = x[j + h];
                    x[j] = a + b;
                    x[j + h] = a - b;
                }
        for (int i = 0; i < 128; ++i) x[i] *= scale;
    }
    return OR_OK;
}

/* =========================================================================================== one weight */

/* common/exl3_decode.c:193-221: W_hat rows of the canonical plane, tile by tile. */
static int what_rows(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int bits, int codebook,
                     int64_t row0, int64_t n, float* outf, uint16_t* outh) {
    uint8_t sym[256];
    uint16_t st[256];
    int tr[256], tc[256];
    if (!codes || (!outf && !outh) || !bits_ok(bits) || !cb_ok(codebook)) return OR_E_ARG;
    if (rows <= 0 || cols <= 0 || rows % 16 || cols % 16 || row0 < 0 || n < 0 || row0 + n > rows) return OR_E_SHAPE;
    if (!row_bytes) row_bytes = or_codes_row_bytes(cols, bits);
    for (int p = 0; p < 256; ++p) or_pos_to_tile(p, &tr[p], &tc[p]);
    for (int64_t tn = row0 / 16; tn * 16 < row0 + n; ++tn)
        for (int64_t tk = 0; tk < cols / 16; ++tk) {
            for (int p = 0; p < 256; ++p)
                sym[p] = (uint8_t)or_codes_get(codes, row_bytes, bits, tn * 16 + tc[p], tk * 16 + tr[p]);
            or_tile_states(sym, bits, st);
            for (int p = 0; p < 256; ++p) {
                const int64_t i = tn * 16 + tc[p];
                if (i < row0 || i >= row0 + n) continue;
                const uint16_t v = or_codebook_value(st[p], codebook);
                const int64_t at = (i - row0) * cols + tk * 16 + tr[p];
                if (outf) outf[at] = or_half_to_float(v);
                if (outh) outh[at] = v;
            }
        }
    return OR_OK;
}

int or_decode_what_rows(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int bits,
                        int codebook, int64_t row0, int64_t n, float* out) {
    return what_rows(codes, row_bytes, rows, cols, bits, codebook, row0, n, out, 0);
}

int or_decode_what_rows_f16(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int bits,
                            int codebook, int64_t row0, int64_t n, uint16_t* out) {
    return what_rows(codes, row_bytes, rows, cols, bits, codebook, row0, n, 0, out);
}

/* common/exl3_decode.c:225-271: W of one 128-row block in exllamav3's order -- had over k (along a row here), x suh
 * (suh1 for the up half of a stacked weight), had over n (down a column), x svh -- then the asked rows copied. */
int or_decode_rows(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int bits, int codebook,
                   const uint16_t* suh, const uint16_t* suh1, const uint16_t* svh, int64_t row0, int64_t n,
                   float* out) {
    if (!codes || !suh || !svh || !out || !bits_ok(bits) || !cb_ok(codebook)) return OR_E_ARG;
    if (rows <= 0 || cols <= 0 || rows % 128 || cols % 128 || (suh1 && rows % 256) || row0 < 0 || n < 0 ||
        row0 + n > rows)
        return OR_E_SHAPE;
    if (n == 0) return OR_OK;
    float* blk = (float*)malloc((size_t)(128 * cols) * sizeof(float));
    float col[128];
    int rc = OR_OK;
    if (!blk) return OR_E_NOMEM;
    for (int64_t b0 = (row0 / 128) * 128; b0 < row0 + n && rc == OR_OK; b0 += 128) {
        rc = what_rows(codes, row_bytes, rows, cols, bits, codebook, b0, 128, blk, 0);
        if (rc != OR_OK) break;
        for (int r = 0; r < 128; ++r) {
            float* row = blk + (int64_t)r * cols;
            const uint16_t* s = (suh1 && b0 + r >= rows / 2) ? suh1 : suh;
            or_had128(row, cols);
            for (int64_t k = 0; k < cols; ++k) row[k] *= or_half_to_float(s[k]);
        }
        for (int64_t k = 0; k < cols; ++k) {
            for (int r = 0; r < 128; ++r) col[r] = blk[(int64_t)r * cols + k];
            or_had128(col, 128);
            for (int r = 0; r < 128; ++r) blk[(int64_t)r * cols + k] = col[r];
        }
        for (int r = 0; r < 128; ++r) {
            const float s = or_half_to_float(svh[b0 + r]);
            for (int64_t k = 0; k < cols; ++k) blk[(int64_t)r * cols + k] *= s;
        }
        const int64_t lo = b0 > row0 ? b0 : row0, hi = (b0 + 128 < row0 + n) ? b0 + 128 : row0 + n;
        memcpy(out + (lo - row0) * cols, blk + (lo - b0) * cols, (size_t)((hi - lo) * cols) * sizeof(float));
    }
    free(blk);
    return rc;
}

/* =========================================================================================== the ops */

static float h2f(uint16_t h) { return or_half_to_float(h); }
static uint16_t f2h(float f) { return or_f32_to_f16(f); }

/* kernels/exl3ref/ref.c:27-32: xr = f16(had(f16(x * s))). */
static void prologue(const float* x, const uint16_t* s, int64_t cols, float* xr) {
    for (int64_t k = 0; k < cols; ++k) xr[k] = h2f(f2h(x[k] * h2f(s[k])));
    or_had128(xr, cols);
    for (int64_t k = 0; k < cols; ++k) xr[k] = h2f(f2h(xr[k]));
}

int or_prologue(const float* x, const uint16_t* s, int64_t n, float* xr) {
    if (!x || !s || !xr || n % 128) return OR_E_SHAPE;
    prologue(x, s, n, xr);
    return OR_OK;
}

/* kernels/exl3ref/ref.c:35-42: acc[n] = sum over ascending k of xr[k] * what[n][k], one product and one add. */
static void gemv(const float* xr, const float* what, int64_t rows, int64_t cols, float* acc) {
    for (int64_t n = 0; n < rows; ++n) {
        const float* w = what + n * cols;
        float s = 0.0f;
        for (int64_t k = 0; k < cols; ++k) {
            const float p = xr[k] * w[k];
            s = s + p;
        }
        acc[n] = s;
    }
}

/* kernels/exl3ref/ref.c:44 */
static float silu(float g) { return g * (1.0f / (1.0f + expf(-g))); }

static const void* tab(const void* base, int64_t stride, int64_t j) { return (const uint8_t*)base + j * stride; }

/* Row r of the input (cols from col0), widened to f32 (kernels/exl3ref/ref.c:142-146). */
static void load_row(const OrOp* o, int64_t r, int64_t col0, int64_t cols, float* out) {
    const uint16_t* p = (const uint16_t*)o->x + r * o->x_pitch + col0;
    for (int64_t k = 0; k < cols; ++k) out[k] = o->x_bf16 ? or_bf16_to_f32(p[k]) : h2f(p[k]);
}

typedef struct Work { float *what, *x, *xr, *acc; } Work;

/* kernels/exl3ref/ref.c:154-169: prep_gu's rows of one run. */
static void prep_rows(const OrOp* o, int64_t e, Work* w) {
    const int c = (int)(e % o->n_class);
    const int64_t j = e / o->n_class, C = o->cls[c].cols;
    const uint16_t* s[2] = { tab(o->cls[c].suh, o->cls[c].suh_stride, j), tab(o->cls[c].suh1, o->cls[c].suh1_stride, j) };
    for (int64_t i = o->expert_offset[e]; i < o->expert_offset[e + 1]; ++i) {
        uint16_t* xr = (uint16_t*)o->y + i * o->y_pitch;
        if (o->sorted_tok[i] < 0) { memset(xr, 0, (size_t)(2 * C) * 2); continue; }
        load_row(o, o->sorted_tok[i] / o->top_k, 0, C, w->x);
        for (int p = 0; p < 2; ++p) {
            prologue(w->x, s[p], C, w->xr);
            for (int64_t k = 0; k < C; ++k) xr[p * C + k] = f2h(w->xr[k]);
        }
    }
}

/* kernels/exl3ref/ref.c:171-228: one live expert's rows of gate_up or down. */
static int expert_rows(const OrOp* o, int64_t e, Work* w) {
    const int c = (int)(e % o->n_class);
    const OrClass* k = &o->cls[c];
    const int64_t R = k->rows, C = k->cols, j = e / o->n_class;
    const int gate_up = o->op == 1;
    const uint16_t* suh = tab(k->suh, k->suh_stride, j);
    const uint16_t* suh1 = gate_up ? tab(k->suh1, k->suh1_stride, j) : 0;
    const uint16_t* svh = tab(k->svh, k->svh_stride, j);
    const uint8_t* codes = tab(k->codes, k->codes_stride, j);
    int rc = or_decode_what_rows(codes, 0, R, C, o->bits, o->codebook, 0, R, w->what);
    if (rc != OR_OK) return rc;
    for (int64_t i = o->expert_offset[e]; i < o->expert_offset[e + 1]; ++i) {
        if (o->sorted_tok[i] < 0) continue;
        if (gate_up) {
            const int64_t W = R / 2;
            uint16_t* h = (uint16_t*)o->y + i * o->y_pitch;
            if (!o->a_rot) load_row(o, o->sorted_tok[i] / o->top_k, 0, C, w->x);
            for (int p = 0; p < 2; ++p) {
                if (o->a_rot) load_row(o, i, p * C, C, w->xr);
                else prologue(w->x, p ? suh1 : suh, C, w->xr);
                gemv(w->xr, w->what + p * W * C, W, C, w->acc + p * W);
                or_had128(w->acc + p * W, W);
                for (int64_t n = 0; n < W; ++n) w->acc[p * W + n] = w->acc[p * W + n] * h2f(svh[p * W + n]);
            }
            if (!o->h_rot) {
                for (int64_t n = 0; n < W; ++n) h[n] = f2h(silu(w->acc[n]) * w->acc[W + n]);
                continue;
            }
            for (int64_t n = 0; n < W; ++n) w->x[n] = h2f(f2h(silu(w->acc[n]) * w->acc[W + n]));
            prologue(w->x, tab(k->dn_suh, k->dn_suh_stride, j), W, w->xr);
            for (int64_t n = 0; n < W; ++n) h[n] = f2h(w->xr[n]);
        } else {
            if (o->h_rot) {
                load_row(o, i, 0, C, w->xr);
            } else {
                load_row(o, i, 0, C, w->x);
                prologue(w->x, suh, C, w->xr);
            }
            gemv(w->xr, w->what, R, C, w->acc);
            or_had128(w->acc, R);
            uint16_t* y = (uint16_t*)o->y + i * o->y_pitch;
            for (int64_t n = 0; n < R; ++n) y[n] = or_f32_to_bf16(w->acc[n] * h2f(svh[n]));
        }
    }
    return OR_OK;
}

static int64_t y_cols_of(const OrOp* o) {
    int64_t x = 0, r = 0;
    for (int c = 0; c < o->n_class; ++c) {
        if (o->cls[c].cols > x) x = o->cls[c].cols;
        if (o->cls[c].rows > r) r = o->cls[c].rows;
    }
    return o->op == 2 ? 2 * x : o->op == 1 ? r / 2 : r;
}

/* Threads or_launch spreads the experts over (OpenMP): 1 unless a caller asks for more. Each expert's rows are one
 * thread's, computed exactly as on one thread, so the bits do not depend on the count. */
static int g_threads = 1;
void or_set_threads(int n) { g_threads = n > 0 ? n : 1; }
int  or_get_threads(void) { return g_threads; }

/* kernels/exl3ref/ref.c:307-331: zero every output row (not prep_gu's), then each live expert's rows once -- the
 * experts independent of each other, so a thread each (one decode of W_hat a live expert, as the reference does). */
int or_launch(const OrOp* o) {
    const int64_t y_cols = y_cols_of(o);
    int64_t most = 0, widest = 0, xc = 0;
    int rc = OR_OK;
    if (o->op != 2)
        for (int64_t i = 0; i < o->T; ++i) memset((uint16_t*)o->y + i * o->y_pitch, 0, (size_t)y_cols * 2);
    for (int c = 0; c < o->n_class; ++c) {
        if (o->cls[c].rows * o->cls[c].cols > most) most = o->cls[c].rows * o->cls[c].cols;
        if (o->cls[c].rows > widest) widest = o->cls[c].rows;
        if (o->cls[c].cols > xc) xc = o->cls[c].cols;
    }
    const int64_t row = xc > widest ? xc : widest;
#pragma omp parallel num_threads(g_threads)
    {
        Work w = { malloc((size_t)(most + 1) * sizeof(float)), malloc((size_t)(row + 1) * sizeof(float)),
                   malloc((size_t)(row + 1) * sizeof(float)), malloc((size_t)(widest + 1) * sizeof(float)) };
        int mine = (!w.what || !w.x || !w.xr || !w.acc) ? OR_E_NOMEM : OR_OK;
#pragma omp for schedule(dynamic, 1)
        for (int64_t e = 0; e < o->n_expert; ++e) {
            if (mine != OR_OK) continue;
            const int64_t lo = o->expert_offset[e], hi = o->expert_offset[e + 1];
            int live = 0;
            for (int64_t i = lo; i < hi && !live; ++i) live = o->sorted_tok[i] >= 0;
            if (o->op == 2) {
                if (hi > lo) prep_rows(o, e, &w);
            } else if (live) {
                mine = expert_rows(o, e, &w);
            }
        }
#pragma omp critical
        if (mine != OR_OK && rc == OR_OK) rc = mine;
        free(w.what); free(w.x); free(w.xr); free(w.acc);
    }
    return rc;
}

int or_gate_up_down(const OrOp* gu, const OrOp* dn) {
    int64_t W = 0;
    for (int c = 0; c < gu->n_class; ++c)
        if (gu->cls[c].rows / 2 > W) W = gu->cls[c].rows / 2;
    const int64_t T = gu->T;
    uint16_t* h = (uint16_t*)calloc((size_t)(T > 0 ? T : 1) * (size_t)W, 2);
    if (!h) return OR_E_NOMEM;
    OrOp g = *gu, d = *dn;
    g.a_rot = 0; g.h_rot = 1; g.y = h; g.y_pitch = W;
    d.h_rot = 1; d.x = h; d.x_bf16 = 0; d.x_rows = T; d.x_pitch = W;
    int rc = or_launch(&g);
    if (rc == OR_OK) rc = or_launch(&d);
    free(h);
    return rc;
}

/* =========================================================================================== routing */

/* include/exl3_abi.h:109-123; tests/ref/exl3_numpy.py:223-242: count per expert, exclusive prefix, then place
 * each flat index in ascending order (stable); a slot outside the owned range is not placed. */
void or_moe_scatter_full(const int32_t* ids, int64_t n_tok, int64_t top_k, int64_t base, int64_t n_expert,
                         int32_t* sorted_tok, int32_t* off, int32_t* count, int32_t* row_of) {
    const int64_t n = n_tok * top_k;
    int64_t* fill = (int64_t*)calloc((size_t)n_expert + 1, sizeof(int64_t));
    for (int64_t e = 0; e <= n_expert; ++e) off[e] = 0;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t e = (int64_t)ids[i] - base;
        if (e >= 0 && e < n_expert) off[e + 1]++;
    }
    if (count)
        for (int64_t e = 0; e < n_expert; ++e) count[e] = off[e + 1];
    for (int64_t e = 0; e < n_expert; ++e) off[e + 1] += off[e];
    for (int64_t i = 0; i < n; ++i) sorted_tok[i] = -1;
    for (int64_t i = 0; i < n; ++i) {
        const int64_t e = (int64_t)ids[i] - base;
        int32_t pos = -1;
        if (e >= 0 && e < n_expert) {
            pos = (int32_t)(off[e] + fill[e]++);
            sorted_tok[pos] = (int32_t)i;
        }
        if (row_of) row_of[i] = pos;
    }
    free(fill);
}

void or_moe_scatter(const int32_t* ids, int64_t n_tok, int64_t top_k, int64_t base, int64_t n_expert,
                    int32_t* sorted_tok, int32_t* off) {
    or_moe_scatter_full(ids, n_tok, top_k, base, n_expert, sorted_tok, off, NULL, NULL);
}

/* a ranks before b: the larger logit, or the same logit and the lower id; a NaN logit after every number */
static int rank_before(float la, int64_t ea, float lb, int64_t eb) {
    const int na = la != la, nb = lb != lb;
    if (na != nb) return nb;
    if (!na && la != lb) return la > lb;
    return ea < eb;
}

void or_router_topk(const float* logits, int64_t n_tok, int64_t n_expert, int64_t pitch, int top_k, int renorm,
                    int32_t* ids, float* w) {
    for (int64_t t = 0; t < n_tok; ++t) {
        const float* l = logits + t * pitch;
        double m = -INFINITY, s = 0.0, sk = 0.0, p[64];
        for (int64_t e = 0; e < n_expert; ++e)
            if (l[e] > m) m = l[e];
        for (int64_t e = 0; e < n_expert; ++e) s += exp((double)l[e] - m);
        float prev_l = 0.f;
        int64_t prev_e = -1;
        for (int j = 0; j < top_k; ++j) {
            int64_t be = -1;
            for (int64_t e = 0; e < n_expert; ++e) {
                if (j > 0 && !rank_before(prev_l, prev_e, l[e], e)) continue;
                if (be < 0 || rank_before(l[e], e, l[be], be)) be = e;
            }
            prev_l = l[be];
            prev_e = be;
            ids[t * top_k + j] = (int32_t)be;
            p[j] = exp((double)l[be] - m) / s;
            sk += p[j];
        }
        for (int j = 0; j < top_k; ++j) w[t * top_k + j] = (float)(renorm ? p[j] / sk : p[j]);
    }
}

static float or_bits_to_f32(uint16_t b, int bf16) {
    if (bf16) {
        const uint32_t u = (uint32_t)b << 16;
        float f;
        memcpy(&f, &u, 4);
        return f;
    }
    return or_half_to_float(b);
}

void or_moe_gather(const uint16_t* y, int y_bf16, int64_t y_pitch, const float* w, const int32_t* row_of,
                   int64_t n_tok, int top_k, int64_t cols, uint16_t* out, int64_t out_pitch) {
    for (int64_t t = 0; t < n_tok; ++t)
        for (int64_t c = 0; c < cols; ++c) {
            float acc = 0.f;
            for (int s = 0; s < top_k; ++s) {
                const int32_t r = row_of[t * top_k + s];
                if (r < 0) continue;
                const float prod = w[t * top_k + s] * or_bits_to_f32(y[(int64_t)r * y_pitch + c], y_bf16);
                acc = acc + prod;
            }
            out[t * out_pitch + c] = or_f32_to_f16(acc);
        }
}
