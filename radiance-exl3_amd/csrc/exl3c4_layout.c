/* exl3c4_layout.c -- the stored form of a codes plane, both directions (host, load time).
 *
 * The canonical plane (include/exl3_encoding.h:12-13) keeps the K-bit symbol of W_hat[k = j][n = i] at element (i, j),
 * each row a bit stream LSB first from bit j K (common/exl3_decode.c:148-168). A tile (tk, tn) of the weight is the
 * MSB-first stream of its 256 symbols in trellis-position order, position p at tile (r, c) = pos_to_tile(p)
 * (common/exl3_decode.c:71-121; common/exl3_layout.c:62-104 is the reference's codes <-> record walk). The stored form
 * of this library cuts every tile's 8 K words into 8 segments of K words (positions 32 s .. 32 s + 31) and places them
 * where the wave that decodes them loads them with one contiguous access (include/exl3c4.h, "THE STORED FORM"):
 *
 *   block (nb, ks) = strip nb of 32 columns x step ks of 64 k, at block index nb * (cols / 64) + ks, 64 K words;
 *   segment X = c + 16 g of the block (c = 2 s + t) = words [s K, s K + K) of tile (tk = 4 ks + g, tn = 2 nb + t).
 *
 * A lossless permutation of the bits; unrelayout is its inverse. Checked both ways against the oracle's record and
 * against the device decode (tests). */
#include <stdint.h>
#include <string.h>

#include "exl3c4.h"

/* Trellis position p = 8 L + j sits at tile row 2 (L % 4) + {0, 1, 8, 9}[j % 4], column L / 4 + 8 (j / 4)
 * (common/exl3_decode.c:71-76). */
#define TILE_R(p) (2 * (((p) >> 3) & 3) + (((p) & 1) | (((p) & 2) << 2)))
#define TILE_C(p) (((p) >> 5) + 8 * (((p) >> 2) & 1))

/* The two directions are written once for a constant K (always inlined into one copy a K, so the tile map, the masks
 * and the shifts fold to constants and the symbol loops unroll): at K = 4 a tile converts in about a tenth of the
 * time of the same loops with K and the map read at run time. */
#define INLINE static inline __attribute__((always_inline))

/* Tile (tk, tn)'s 8 K stream words from the plane: its 16 rows' 2 K bytes each, symbols LSB first, then the stream
 * (MSB first: position 0 in the top bits of word 0). */
INLINE void tile_words(const uint8_t* codes, int64_t rb, int64_t tk, int64_t tn, const int bits, uint32_t* w) {
    uint8_t sym[16][16];   /* [c][r]: row n = 16 tn + c, column k = 16 tk + r */
    const uint32_t mask = (1u << bits) - 1u;
    const int seg = 2 * bits;
    for (int c = 0; c < 16; ++c) {
        uint8_t b[18] = { 0 };
        memcpy(b, codes + (tn * 16 + c) * rb + tk * seg, (size_t)seg);
        uint64_t lo = 0, hi = 0;                          /* the row's 16 K bits, little-endian */
        memcpy(&lo, b, 8);
        memcpy(&hi, b + 8, 8);
        for (int r = 0; r < 16; ++r) {
            const int o = r * bits;
            const uint64_t v = o < 64 ? (lo >> o) | (o > 0 && o + bits > 64 ? hi << (64 - o) : 0) : hi >> (o - 64);
            sym[c][r] = (uint8_t)(v & mask);
        }
    }
    for (int s = 0; s < 8; ++s) {                         /* segment s: positions 32 s .. 32 s + 31, K words */
        uint64_t acc = 0;
        int nb = 0;
        for (int p = 32 * s; p < 32 * s + 32; ++p) {
            acc = (acc << bits) | sym[TILE_C(p)][TILE_R(p)];
            nb += bits;
            if (nb >= 32) {
                nb -= 32;
                *w++ = (uint32_t)(acc >> nb);
                acc &= (1ull << nb) - 1ull;
            }
        }
    }
}

INLINE void words_tile(const uint32_t* w, int64_t tk, int64_t tn, const int bits, uint8_t* codes, int64_t rb) {
    uint8_t sym[16][16];
    const uint32_t mask = (1u << bits) - 1u;
    for (int s = 0; s < 8; ++s) {
        uint64_t acc = 0;
        int nb = 0;
        for (int p = 32 * s; p < 32 * s + 32; ++p) {
            if (nb < bits) {
                acc = (acc << 32) | *w++;
                nb += 32;
            }
            nb -= bits;
            sym[TILE_C(p)][TILE_R(p)] = (uint8_t)((acc >> nb) & mask);
            acc &= (1ull << nb) - 1ull;
        }
    }
    const int seg = 2 * bits;
    for (int c = 0; c < 16; ++c) {
        uint64_t lo = 0, hi = 0;
        for (int r = 0; r < 16; ++r) {
            const int o = r * bits;
            const uint64_t v = sym[c][r];
            if (o < 64) {
                lo |= v << o;
                if (o + bits > 64) hi |= v >> (64 - o);
            } else {
                hi |= v << (o - 64);
            }
        }
        uint8_t b[16];
        memcpy(b, &lo, 8);
        memcpy(b + 8, &hi, 8);
        memcpy(codes + (tn * 16 + c) * rb + tk * seg, b, (size_t)seg);
    }
}

int64_t exl3c4_record_bytes(int64_t rows, int64_t cols, int32_t bits) { return rows * cols * bits / 8; }

static int shape_ok(int64_t rows, int64_t cols, int bits) {
    return bits >= 1 && bits <= 8 && rows > 0 && cols > 0 && rows % 32 == 0 && cols % 64 == 0;
}

/* Word offset of segment s of tile (tk, tn) in the stored record. */
static int64_t seg_at(int64_t tk, int64_t tn, int s, int64_t ksteps, int bits) {
    const int64_t nb = tn >> 1, ks = tk >> 2;
    const int t = (int)(tn & 1), g = (int)(tk & 3);
    const int X = (2 * s + t) + 16 * g;
    return ((nb * ksteps + ks) * 64 + X) * bits;
}

INLINE void relayout_k(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, const int bits,
                       uint32_t* out) {
    uint32_t w[64];
    const int64_t ksteps = cols / 64;
    for (int64_t tn = 0; tn < rows / 16; ++tn)
        for (int64_t tk = 0; tk < cols / 16; ++tk) {
            tile_words(codes, row_bytes, tk, tn, bits, w);
            for (int s = 0; s < 8; ++s) memcpy(out + seg_at(tk, tn, s, ksteps, bits), w + s * bits, (size_t)bits * 4);
        }
}

INLINE void unrelayout_k(const uint32_t* in, int64_t rows, int64_t cols, const int bits, uint8_t* codes,
                         int64_t row_bytes) {
    uint32_t w[64];
    const int64_t ksteps = cols / 64;
    for (int64_t tn = 0; tn < rows / 16; ++tn)
        for (int64_t tk = 0; tk < cols / 16; ++tk) {
            for (int s = 0; s < 8; ++s) memcpy(w + s * bits, in + seg_at(tk, tn, s, ksteps, bits), (size_t)bits * 4);
            words_tile(w, tk, tn, bits, codes, row_bytes);
        }
}

#define BY_K(CALL)                                                                                                   \
    switch (bits) {                                                                                                  \
    case 1: CALL(1); break;                                                                                          \
    case 2: CALL(2); break;                                                                                          \
    case 3: CALL(3); break;                                                                                          \
    case 4: CALL(4); break;                                                                                          \
    case 5: CALL(5); break;                                                                                          \
    case 6: CALL(6); break;                                                                                          \
    case 7: CALL(7); break;                                                                                          \
    default: CALL(8); break;                                                                                         \
    }

int exl3c4_relayout(const uint8_t* codes, int64_t row_bytes, int64_t rows, int64_t cols, int32_t bits, void* record) {
    if (!codes || !record) return EXL3C4_E_INVAL;
    if (!shape_ok(rows, cols, bits)) return bits < 1 || bits > 8 ? EXL3C4_E_DTYPE : EXL3C4_E_SHAPE;
    if (!row_bytes) row_bytes = (cols * bits + 7) / 8;
    if (row_bytes < (cols * bits + 7) / 8) return EXL3C4_E_STRIDE;
#define RL(K) relayout_k(codes, row_bytes, rows, cols, K, (uint32_t*)record)
    BY_K(RL)
#undef RL
    return EXL3C4_OK;
}

int exl3c4_unrelayout(const void* record, int64_t rows, int64_t cols, int32_t bits, uint8_t* codes, int64_t row_bytes) {
    if (!codes || !record) return EXL3C4_E_INVAL;
    if (!shape_ok(rows, cols, bits)) return bits < 1 || bits > 8 ? EXL3C4_E_DTYPE : EXL3C4_E_SHAPE;
    if (!row_bytes) row_bytes = (cols * bits + 7) / 8;
    if (row_bytes < (cols * bits + 7) / 8) return EXL3C4_E_STRIDE;
#define URL(K) unrelayout_k((const uint32_t*)record, rows, cols, K, codes, row_bytes)
    BY_K(URL)
#undef URL
    return EXL3C4_OK;
}

/* exllamav3's tile record -- int16 [cols / 16][rows / 16][16 K], tk outer, a tile its 8 K stream words, each word two
 * int16 little-endian (common/exl3_layout.c:38-56, common/exl3_decode.c:85-88) -- into the canonical plane: the trellis
 * tensor of a checkpoint as the import (exl3c4_import.c) takes it. */
INLINE void record_codes_k(const uint16_t* rec, int64_t rows, int64_t cols, const int bits, uint8_t* codes,
                           int64_t row_bytes) {
    uint32_t w[64];
    const int64_t nt = rows / 16, kt = cols / 16;
    for (int64_t tk = 0; tk < kt; ++tk)
        for (int64_t tn = 0; tn < nt; ++tn) {
            const uint16_t* t = rec + (tk * nt + tn) * 16 * bits;
            for (int q = 0; q < 8 * bits; ++q) w[q] = (uint32_t)t[2 * q] | ((uint32_t)t[2 * q + 1] << 16);
            words_tile(w, tk, tn, bits, codes, row_bytes);
        }
}

int exl3c4_record_to_codes(const uint16_t* record, int64_t rows, int64_t cols, int32_t bits, uint8_t* codes,
                           int64_t row_bytes) {
    if (!codes || !record) return EXL3C4_E_INVAL;
    if (bits < 1 || bits > 8) return EXL3C4_E_DTYPE;
    if (rows <= 0 || cols <= 0 || rows % 16 || cols % 16) return EXL3C4_E_SHAPE;
    if (!row_bytes) row_bytes = (cols * bits + 7) / 8;
    if (row_bytes < (cols * bits + 7) / 8) return EXL3C4_E_STRIDE;
#define RC(K) record_codes_k(record, rows, cols, K, codes, row_bytes)
    BY_K(RC)
#undef RC
    return EXL3C4_OK;
}
