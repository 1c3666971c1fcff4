// exl3c4_dev.hip -- the gfx950 (CDNA4, wave64) kernels of exl3c4 and their extern "C" launchers.
//
// The work, per the reference's op contract (docs/OPS-exl3.md:84-153):
//   prep      xr = f16(had128(f16(x * suh)))  per sorted row and half          (kernels/exl3ref/ref.c:27-32, 154-169)
//   gemv      acc[n] = sum_k xr[k] * W_hat[n][k]: the bitshift-trellis decode of the stored record in registers,
//             fed straight into v_mfma_f32_16x16x32_f16                          (kernels/exl3ref/ref.c:35-42)
//   epilogue  had128 over each 128 output columns, x svh, SiLU(gate) * up -> f16 (optionally rotated again for
//             down, "h_rot"), or -> bf16 for down                              (kernels/exl3ref/ref.c:187-225)
//   dequant   W_hat itself, through the same decode                            (common/exl3_decode.c:193-221)
//
// THE MFMA MAPPING. One wave step covers 4 k-tiles x 2 n-tiles (a 64 x 32 block of W_hat, 2048 weights) with four
// v_mfma_f32_16x16x32_f16: tokens are the MFMA's M (rows), weight columns its N. Lane X = c + 16 g (c = 2 s + t)
// decodes segment s (positions 32 s .. 32 s + 31, i.e. stream words [s K, s K + K)) of tile (tk = 4 ks + g,
// tn = 2 nb + t). Trellis position p = 8 L + j sits at tile row 2 (L % 4) + {0,1,8,9}[j % 4] and column
// L / 4 + 8 (j / 4) (common/exl3_decode.c:71-76), so a segment holds column s (j < 4) and column s + 8 (j >= 4), 16 k
// each, in runs of four -- the lane's B operands of the four MFMAs. The A operand (activations) is read in the
// matching k order, which for the four-run pattern is a pure choice of dwords out of two 16-byte loads.
//
// THE DECODE (codebook mul1, the path's codebook). The state of position q is the 16-bit window of the segment's
// stream ending at bit (q + 1) K, taken from the segment's K words and the previous segment's last word (one DPP
// row_ror:2, the previous segment of the same tile sitting two lanes down, circularly). One v_alignbit_b32 yields a
// register whose low half is one state and (for K | 16) whose high half is another; the hash x * 0x83DCD12D mod 2^32
// is v_pk_mul_lo_u16 (the high partial product, placed in the high half by op_sel) + v_mad_u32_u16 (op_sel picks the
// state's half), so no state is ever masked; the byte sum lands as fp16 bits 0x6400 + s through v_sad_u8 /
// v_sad_hi_u8 for two weights at once, and one v_pk_fma_f16 forms (1024 + s) * K_INV + K_BIAS for both with one
// rounding each -- exactly common/exl3_decode.c:47-58.
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>

#include <stdint.h>
#include <string.h>
#include <utility>

#include "exl3c4_dev.h"

static_assert(sizeof(Exl3c4Launch) == EXL3C4_KERNARG_BYTES && EXL3C4_KERNARG_BYTES <= EXL3C4_KERNARG_LIMIT,
              "the op kernels' argument block must fit the engine's kernel-argument slot");

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef unsigned short ushort2_t __attribute__((ext_vector_type(2)));
typedef float    float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a_t __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x3a_t __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x2a_t __attribute__((ext_vector_type(2), aligned(4)));

constexpr float kHadScale = 0.08838834764831844055f;   // (float)(1/sqrt(128)), common/exl3_decode.c:173

// ------------------------------------------------------------------------------------------------ scalar helpers

// Entry j of a per-expert table: base + j x stride, or with stride 0 the j-th pointer of a pointer table. The table
// is read as constant memory (it does not change during a launch), so a uniform j is a scalar load, counted apart
// from the vector loads: the vector loads in flight around it (codes, activations) are not waited for at the join.
typedef const void* cvptr;
__device__ __forceinline__ const void* tab_entry(const void* base, int32_t stride, int64_t j) {
    return stride ? (const void*)((const char*)base + j * (int64_t)stride)
                  : ((const __attribute__((address_space(4))) cvptr*)base)[j];
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// f32 -> f16, round to nearest even, of an f32 VALUE. The empty asm makes the operand a materialised f32 register:
// without it the backend folds a producing multiply into v_fma_mixlo_f16, which rounds the exact product to f16 once,
// where the reference rounds it to f32 first (a tie then lands on the other side, as measured on gfx950).
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
// Two f32 VALUES -> f16 (lo in the low half), each rounded to nearest even: one v_cvt_pk_f16_f32 (gfx950), the
// operands materialised as f2h's are.
__device__ __forceinline__ uint32_t f2h2(float lo, float hi) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
    asm volatile("" : "+v"(lo), "+v"(hi));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){ lo, hi }, f16x2_t));
}
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
// Two f32 to bf16 (lo in the low half): round to nearest even on the f32 bits, a nan kept quiet as (u >> 16) | 0x40
// (radiance's rad_f32_to_bf16). One v_cvt_pk_bf16_f32 (gfx950), which gives those bits for every f32: compared on
// the device over each of the 65,536 upper halves with the low halves 0, 1, 0x7FFF, 0x8000, 0x8001 and 0xFFFF (every
// nan class, the ties, the denormals) and 4 M random values, without a difference.
__device__ __forceinline__ uint32_t f2bf2(float lo, float hi) {
    typedef float f32x2_t __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){ lo, hi }, bf16x2_t));
}

// The element of a 128-block that lane l holds for the Hadamard (v0; v1 holds that + 64): l with bits 0 and 1
// flipped where bit 2 is set. Then the partners of every stage up to h = 8 are DPP lanes: element j ^ 1, j ^ 2 at
// lane l ^ 1, l ^ 2 (quad_perm), j ^ 4 at l ^ 7 (row_half_mirror), j ^ 8 at l ^ 8 (row_ror 8). had128_wave<false>
// takes a block in this layout and leaves it in had_col_t's (bits 4 and 5 of the element exchanged), and
// had128_wave<true> the other way round. Every kernel loads, scales and stores a block's values at the elements of
// its layout, so the maps change no value.
__device__ __forceinline__ int had_col(int lane) { return lane ^ (((lane >> 2) & 1) * 3); }
__device__ __forceinline__ int had_col_t(int lane) {
    const int j = had_col(lane);
    return (j & ~48) | ((j & 16) << 1) | ((j & 32) >> 1);
}

// The normalised Sylvester Hadamard over one 128-block held by a wave: the butterfly stages h = 1 .. 64 in the
// reference's order, each (a + b) low and (a - b) high in f32, then one f32 multiply by 1/sqrt(128)
// (common/exl3_decode.c:172-189) -- the same roundings, so the same values. Bits 0..3 of an element sit in bits 0..3 of
// its lane (had_col); bits 4, 5 and 6 in lane bit 4, lane bit 5 and the register (v0, v1), in an order each stage
// from h = 16 on changes. For h = 1, 2, 4, 8 the stage is one v_fmac_f32 whose partner operand comes by DPP:
// v += c p with c = -1 where bit h of the element is set, which leaves those lanes the NEGATED result
// (v - p = -(p - v)); a partner's element has the same lower bits, hence the same sign, so c needs no correction,
// and the signs are undone by the final multiply (by -1/sqrt(128) where an odd number of the bits 1, 2, 4, 8 of the
// element are set). Negation is exact, so every nonzero result is the reference's bits; an exact zero is not
// negated by the trick (v - p = +0 where v = p, whose negation would be -0), so the final step is
// fma(v, +-1/sqrt(128), +0), which gives every zero output +0. That is the reference's zero wherever any of the
// block's 128 inputs is nonzero (values not all zero that cancel sum to +0 in round-to-nearest, and a stage makes -0
// only from two zero operands); a block of 128 zeros rotates to +0 throughout, where the reference's exact-sign
// stages can leave -0 at some outputs (the same value, the other sign bit). For h = 16, 32, 64 one permlane swap of
// v0 and v1 (gfx950: VDST's odd 16-lane rows with SRC0's even rows, or VDST's upper 32 lanes with SRC0's lower ones)
// brings the stage's bit from the lane into the register, so the pair sits in one lane and the stage is an add and a
// subtract; the bit the register held goes to the lane. The DPP and swap stages run with the whole wave active: every caller's branch around them is uniform.
#define HAD_DPP(v, c, CTRL) asm volatile("s_nop 1\n\tv_fmac_f32_dpp %0, %0, %1 " CTRL " row_mask:0xf bank_mask:0xf" \
                                         : "+v"(v) : "v"(c))
// v0 and v1 exchanged across 16-lane rows (W = 16) or 32-lane halves (W = 32): a lane of the odd row (upper half)
// takes the partner lane's v1 into its v0, a lane of the even row (lower half) its partner's v0 into its v1.
template <int W> __device__ __forceinline__ void swap_rows(float& v0, float& v1) {
    const unsigned a = __builtin_bit_cast(unsigned, v0), b = __builtin_bit_cast(unsigned, v1);
    unsigned na, nb;
    if constexpr (W == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(a, b, false, false);
        na = r[0]; nb = r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(a, b, false, false);
        na = r[0]; nb = r[1];
    }
    v0 = __builtin_bit_cast(float, na);
    v1 = __builtin_bit_cast(float, nb);
}
// T_IN = false: in had_col's layout (element bits 4, 5, 6 in lane bit 4, lane bit 5, the register), out in
// had_col_t's (lane bit 5, lane bit 4, the register); T_IN = true the other way round.
template <bool T_IN> __device__ __forceinline__ void had128_wave(float& v0, float& v1, int lane) {
    const int j = had_col(lane);                                  // the element's bits 0..3, in either layout
    const float c1 = (j & 1) ? -1.f : 1.f, c2 = (j & 2) ? -1.f : 1.f, c4 = (j & 4) ? -1.f : 1.f;
    const float c8 = (j & 8) ? -1.f : 1.f;
    HAD_DPP(v0, c1, "quad_perm:[1,0,3,2]");
    HAD_DPP(v1, c1, "quad_perm:[1,0,3,2]");
    HAD_DPP(v0, c2, "quad_perm:[2,3,0,1]");
    HAD_DPP(v1, c2, "quad_perm:[2,3,0,1]");
    HAD_DPP(v0, c4, "row_half_mirror");
    HAD_DPP(v1, c4, "row_half_mirror");
    HAD_DPP(v0, c8, "row_ror:8");
    HAD_DPP(v1, c8, "row_ror:8");
    float a, b;
    swap_rows<T_IN ? 32 : 16>(v0, v1);                            // h = 16: bit 4 into the register
    a = v0 + v1;
    b = v0 - v1;
    v0 = a;
    v1 = b;
    swap_rows<T_IN ? 16 : 32>(v0, v1);                            // h = 32: bit 5 into the register
    a = v0 + v1;
    b = v0 - v1;
    v0 = a;
    v1 = b;
    swap_rows<T_IN ? 32 : 16>(v0, v1);                            // h = 64: bit 6 back into the register
    a = v0 + v1;
    b = v0 - v1;
    const float sc = (__builtin_popcount(j & 15) & 1) ? -kHadScale : kHadScale;
    v0 = __builtin_fmaf(a, sc, 0.f);                              // + 0: an exact zero leaves as +0 (see HAD_DPP)
    v1 = __builtin_fmaf(b, sc, 0.f);
}

// The expert owning sorted row i -- e with off[e] <= i < off[e + 1], or -1 (include/exl3_abi.h:136-141) -- found
// by a whole wave at once: the number of e in [1, n_expert] with off[e] <= i, counted over
// one round of independent loads and a wave reduction, checked against off[e] <= i < off[e + 1] (-1 otherwise). A
// dependent binary search costs one memory latency per halving; this costs about one in all.
__device__ __forceinline__ int owner_wave(const int32_t* off, int n_expert, int i, int lane) {
    constexpr int OJ = 9;                                         // up to 575 experts: one round of loads
    if (n_expert < 64 * OJ) {
        // off[0 .. n_expert] held by the wave (lane l, register j: e = l + 64 j, past n_expert a copy of the last),
        // loaded at once; the owner's number counted by ballots (a scalar result); off[e] and off[e + 1] then read
        // out of the registers, not loaded again
        int o[OJ];
#pragma unroll
        for (int j = 0; j < OJ; ++j) o[j] = off[min(lane + 64 * j, n_expert)];
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < OJ; ++j) {
            const int e = lane + 64 * j;
            cnt += __popcll(__ballot(e >= 1 && e <= n_expert && o[j] <= i));
        }
        const int e = min(cnt, n_expert - 1);
        int lo = 0, hi = 0;
#pragma unroll
        for (int j = 0; j < OJ; ++j) {                            // uniform tests: the registers that hold them
            if ((e >> 6) == j) lo = __builtin_amdgcn_readlane(o[j], e & 63);
            if (((e + 1) >> 6) == j) hi = __builtin_amdgcn_readlane(o[j], (e + 1) & 63);
        }
        return (lo <= i && i < hi) ? e : -1;
    }
    int cnt = 0;
#pragma unroll 8
    for (int e = 1 + lane; e <= n_expert; e += 64) cnt += off[e] <= i ? 1 : 0;
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) cnt += __shfl_xor(cnt, d);
    const int e = min(cnt, n_expert - 1);
    return (off[e] <= i && i < off[e + 1]) ? e : -1;
}

// ------------------------------------------------------------------------------------------------ the decode

struct Mul1Consts {
    uint32_t kh;      // 0x83DC in the high half: v_pk_mul_lo_u16 puts x * 0x83DC there, zero in the low half
    uint32_t cl;      // 0xD12D: the low 16 bits of the multiplier
    uint32_t c6464;   // fp16 1024.0 in both halves: the byte sums add onto it
    half2_t  kinv, kbias;
};

__device__ __forceinline__ Mul1Consts mul1_consts() {
    Mul1Consts k;
    k.kh = 0x83DC0000u;
    k.cl = 0x0000D12Du;
    k.c6464 = 0x64006400u;
    k.kinv = half2_t{ __builtin_bit_cast(_Float16, (uint16_t)0x1EEEu), __builtin_bit_cast(_Float16, (uint16_t)0x1EEEu) };
    k.kbias = half2_t{ __builtin_bit_cast(_Float16, (uint16_t)0xC931u), __builtin_bit_cast(_Float16, (uint16_t)0xC931u) };
    return k;
}

// Two states (in half HA of ra and half HB of rb) -> their two fp16 weights in one dword, low half from ra's. Per
// state: h = x * 0x83DCD12D mod 2^32 = (x * 0x83DC mod 2^16) << 16 + x * 0xD12D -- v_pk_mul_lo_u16 puts the high
// partial product in the high half over a zero low half (op_sel), v_mad_u32_u16 adds x * 0xD12D reading only the
// state's half (op_sel), so no state is masked. Then v_sad_u8 / v_sad_hi_u8 leave 0x6400 + bytesum in each half
// (fp16 1024 + s, exact), and one v_pk_fma_f16 forms (1024 + s) * K_INV + K_BIAS for both, one rounding each.
// Only the two v_mad_u32_u16 are asm (their op_sel half select is not reached from ordinary code, which spends a
// shift or a mask on it), and they rewrite registers the compiler's own v_pk_mul_lo_u16 defined: the compiler keeps
// every register an MFMA reads in its hazard windows -- a VALU write of an MFMA source needs two wait states before
// the MFMA reads it, and one of a source C the MFMA has read needs three -- only for instructions it emitted, so no
// asm output may be a register first written by the asm or a value an MFMA reads.
template <int H> __device__ __forceinline__ uint32_t mul1_hi_product(uint32_t r, uint32_t kh) {
    const ushort2_t v = __builtin_bit_cast(ushort2_t, r);
    return __builtin_bit_cast(uint32_t, __builtin_shufflevector(v, v, H, H) * __builtin_bit_cast(ushort2_t, kh));
}

template <int HA, int HB>
__device__ __forceinline__ uint32_t mul1_pair(uint32_t ra, uint32_t rb, const Mul1Consts& k) {
    uint32_t ya = mul1_hi_product<HA>(ra, k.kh), yb = mul1_hi_product<HB>(rb, k.kh);
    asm("v_mad_u32_u16 %[ya], %[ra], %[cl], %[ya] op_sel:[%c[ha],0,0,0]\n\t"
        "v_mad_u32_u16 %[yb], %[rb], %[cl], %[yb] op_sel:[%c[hb],0,0,0]"
        : [ya] "+v"(ya), [yb] "+v"(yb)
        : [ra] "v"(ra), [rb] "v"(rb), [cl] "s"(k.cl), [ha] "n"(HA), [hb] "n"(HB));
    const uint32_t s = __builtin_amdgcn_sad_hi_u8(yb, 0u, __builtin_amdgcn_sad_u8(ya, 0u, k.c6464));
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_fma(__builtin_bit_cast(half2_t, s), k.kinv, k.kbias));
}

// mcg / 3inst (common/exl3_decode.c:59-66): a 32-bit hash, (h & 0x8FFF8FFF) ^ 0x3B603B60, fp16 lo + hi rounded once.
template <int CB, int H> __device__ __forceinline__ uint16_t lop_value(uint32_t r) {
    uint32_t x = H ? (r >> 16) : (r & 0xFFFFu);
    x = CB == EXL3C4_CB_MCG ? x * 0xCBAC1FEDu : x * 89226354u + 64248484u;
    x = (x & 0x8FFF8FFFu) ^ 0x3B603B60u;
    const _Float16 s = __builtin_bit_cast(_Float16, (uint16_t)(x & 0xFFFFu)) +
                       __builtin_bit_cast(_Float16, (uint16_t)(x >> 16));
    return __builtin_bit_cast(uint16_t, s);
}

// The window of one segment as K + 1 words from least significant: v[0] = the segment's last word .. v[K - 1] its
// first, v[K] the previous segment's last word. The state of segment position q is window bits [K (31 - q), +16).
template <int BITS, int Q> __device__ __forceinline__ uint32_t state_reg(const uint32_t (&v)[BITS + 1]) {
    constexpr int sh = BITS * (31 - Q);
    constexpr int base = (sh % 32 >= 16) ? sh - 16 : sh;
    constexpr int wb = base / 32, rb = base % 32;
    if constexpr (rb == 0) return v[wb];
    else return __builtin_amdgcn_alignbit(v[wb + 1], v[wb], rb);
}
template <int BITS, int Q> constexpr int state_half() { return (BITS * (31 - Q)) % 32 >= 16 ? 1 : 0; }

// Segment positions Q, Q + 1 (Q even) -> their dword of the B operands. Position q = 8 l + j: register
// R = 2 (j / 4) + l / 2 (B_a, B_b: column s; B_c, B_d: column s + 8), dword 2 (l % 2) + (j % 4) / 2, half j % 2.
template <int BITS, int CB, int Q>
__device__ __forceinline__ void decode_pair(const uint32_t (&v)[BITS + 1], uint32_t (&B)[16], const Mul1Consts& k) {
    const uint32_t ra = state_reg<BITS, Q>(v), rb = state_reg<BITS, Q + 1>(v);
    constexpr int ha = state_half<BITS, Q>(), hb = state_half<BITS, Q + 1>();
    uint32_t out;
    if constexpr (CB == EXL3C4_CB_MUL1) {
        out = mul1_pair<ha, hb>(ra, rb, k);
    } else {
        out = (uint32_t)lop_value<CB, ha>(ra) | ((uint32_t)lop_value<CB, hb>(rb) << 16);
    }
    constexpr int l = Q >> 3, j = Q & 7, jj = j & 3;
    constexpr int R = 2 * (j >> 2) + (l >> 1), dw = 2 * (l & 1) + (jj >> 1);
    B[R * 4 + dw] = out;
}

template <int BITS, int CB, int... P>
__device__ __forceinline__ void decode_seg_impl(const uint32_t (&v)[BITS + 1], uint32_t (&B)[16], const Mul1Consts& k,
                                                std::integer_sequence<int, P...>) {
    (decode_pair<BITS, CB, 2 * P>(v, B, k), ...);
}

// A lane's segment as its decode window (decode_pair's v): the K words reversed, then the previous segment of the same
// tile's last word -- two lanes down, circularly within the 16-lane row (c = 2 s + t).
template <int BITS>
__device__ __forceinline__ void segment_window(const uint32_t (&d)[BITS], uint32_t (&v)[BITS + 1]) {
#pragma unroll
    for (int w = 0; w < BITS; ++w) v[w] = d[BITS - 1 - w];
    v[BITS] = (uint32_t)__builtin_amdgcn_mov_dpp((int)d[BITS - 1], 0x122, 0xF, 0xF, false);
}

// One lane's segment -> its 32 weights as the four B operands (B[0..3] B_a, [4..7] B_b, [8..11] B_c, [12..15] B_d).
template <int BITS, int CB>
__device__ __forceinline__ void decode_segment(const uint32_t (&d)[BITS], uint32_t (&B)[16], const Mul1Consts& k) {
    uint32_t v[BITS + 1];
    segment_window<BITS>(d, v);
    decode_seg_impl<BITS, CB>(v, B, k, std::make_integer_sequence<int, 16>{});
}

// A lane's K words of one block: K u32 at p (4-byte aligned).
template <int BITS, typename P> __device__ __forceinline__ void load_words(P p, uint32_t (&d)[BITS]) {
    typedef __attribute__((address_space(1))) const u32x4a_t* q4p;
    typedef __attribute__((address_space(1))) const u32x3a_t* q3p;
    typedef __attribute__((address_space(1))) const u32x2a_t* q2p;
    int w = 0;
#pragma unroll
    for (; w + 4 <= BITS; w += 4) {
        const u32x4a_t q = *(q4p)(p + w);
        d[w] = q.x; d[w + 1] = q.y; d[w + 2] = q.z; d[w + 3] = q.w;
    }
    if constexpr (BITS % 4 == 3) {
        const u32x3a_t q = *(q3p)(p + w);
        d[w] = q.x; d[w + 1] = q.y; d[w + 2] = q.z;
    } else if constexpr (BITS % 4 == 2) {
        const u32x2a_t q = *(q2p)(p + w);
        d[w] = q.x; d[w + 1] = q.y;
    } else if constexpr (BITS % 4 == 1) {
        d[w] = p[w];
    }
}

__device__ __forceinline__ half8_t as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(half8_t, u32x4_t{ a, b, c, d });
}

// gfx950's v_mfma_f32_16x16x32_f16 still reads its A and B registers for some cycles after it issues, and the compiler
// does not hold back a VALU or load that writes them meanwhile (measured: an address computed into a just-issued MFMA's
// B registers corrupted the product). Every group of MFMAs ends with this guard: the scheduler may move nothing across
// it, and its inputs keep the group's operand registers allocated through 16 wait states after the last MFMA.
__device__ __forceinline__ void mfma_guard(const half8_t& a0, const half8_t& a1, const half8_t& b0, const half8_t& b1,
                                           const half8_t& b2, const half8_t& b3) {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n\ts_nop 7" ::"v"(a0), "v"(a1), "v"(b0), "v"(b1), "v"(b2), "v"(b3));
    __builtin_amdgcn_sched_barrier(0);
}

// ------------------------------------------------------------------------------------------------ kernels

// The order of k inside every 16-group of an activation row stored PERMUTED: position p holds k = kPerm[p], so that one
// 16-byte load is the A operand of the first two MFMAs of a step (k 0,1,8,9,2,3,10,11) and the next 16 bytes the
// second two (4,5,12,13,6,7,14,15) -- the trellis segment's run pattern. kSlot is its inverse (where k is stored).
// Expert e's class and its entry in the class's tables: experts interleave over the classes (n_class is 1, 2 or 4).
__device__ __forceinline__ int class_of(const Exl3c4Launch& a, int e) { return e & (a.n_class - 1); }
__device__ __forceinline__ int64_t entry_of(const Exl3c4Launch& a, int e) { return e >> (a.n_class >> 1); }

__device__ __forceinline__ int perm_slot(int k) {
    const int q = k & 15;
    const int slot = ((q & 1) | ((q >> 3) << 1)) + (((q >> 1) & 1) << 2) + (((q >> 2) & 1) << 3);
    return (k & ~15) | slot;
}

// The owner of sorted row i and its run (include/exl3_abi.h:136-141), found by a whole workgroup in ONE round of
// independent loads: its threads read off[0 .. n_expert] (four entries a thread in flight together, the addresses
// clamped so that no load sits behind a branch), count by wave ballots the e >= 1 with off[e] <= i (for sorted
// offsets, the owner's number) and keep the offsets in LDS, so the run's bounds off[e], off[e + 1] come from there
// after the barrier instead of a second round of loads (up to OWNER_LDS experts; beyond, from memory). The row has an
// owner when e < n_expert and off[e] <= i < off[e + 1]; else -1. lo / hi: the run clamped to [0, T)
// (kernels/exl3r4d/launch.c:14-15). The result is uniform (in scalar registers): the class tables it selects are read
// with scalar loads. Holds a barrier: every thread of the workgroup calls it.
struct Owner { int e, lo, hi; };
constexpr int OWNER_LDS = 1024;
__device__ Owner owner_wg(const Exl3c4Launch& a, int i) {
    __shared__ int cnt_s[4];
    __shared__ int off_s[OWNER_LDS + 1];
    const int n = a.n_expert, tid = (int)threadIdx.x;
    int cnt = 0;
    for (int e0 = 0; e0 <= n; e0 += 4 * 256) {                    // uniform trip count: ballots see every lane
        int o[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) o[j] = a.off[min(e0 + 256 * j + tid, n)];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int e = e0 + 256 * j + tid;
            if (e <= OWNER_LDS && e <= n) off_s[e] = o[j];
            cnt += __popcll(__ballot(e >= 1 && e <= n && o[j] <= i));
        }
    }
    if ((tid & 63) == 0) cnt_s[tid >> 6] = cnt;
    __syncthreads();
    const int e = __builtin_amdgcn_readfirstlane(min(cnt_s[0] + cnt_s[1] + cnt_s[2] + cnt_s[3], n - 1));
    const int o0 = __builtin_amdgcn_readfirstlane(e + 1 <= OWNER_LDS ? off_s[e] : a.off[e]);
    const int o1 = __builtin_amdgcn_readfirstlane(e + 1 <= OWNER_LDS ? off_s[e + 1] : a.off[e + 1]);
    Owner w;
    w.e = (o0 <= i && i < o1) ? e : -1;
    w.lo = max(o0, 0);
    w.hi = min(o1, a.T);
    return w;
}

// A chunk is at most a.chunk_rows rows of one run (a power of two), cut from the run's first row: the workgroup keyed
// on the chunk's first row does the chunk. Rows of the chunk: 0 when row i does not start one. (Where the runs are
// cut changes no bits: every row's products are its own MFMA row.)
__device__ __forceinline__ int chunk_rows(const Exl3c4Launch& a, const Owner& w, int i) {
    const int ch = a.chunk_rows;
    return (w.e >= 0 && ((i - w.lo) & (ch - 1)) == 0) ? min(ch, w.hi - i) : 0;
}

// A lane's row of the staged chunk as the MFMA's A operand reads it: rows past the chunk's staged rows (whose
// products are never written) read the last staged row, so no read leaves the workgroup's LDS.
__device__ __forceinline__ int a_row(const Exl3c4Launch& a, int lane) { return min(lane & 15, a.chunk_rows - 1); }

// f16(had128(f16(v * s))) over one 128-block, lane l holding k = had_col(l) (0) and + 64 (1) of v and s, and
// leaving k = had_col_t(l) and + 64 of the result (kernels/exl3ref/ref.c:27-32).
__device__ __forceinline__ void rotate_block(float f0, float f1, uint16_t s0, uint16_t s1, int lane, uint16_t& o0,
                                             uint16_t& o1) {
    float v0 = h2f(f2h(f0 * h2f(s0))), v1 = h2f(f2h(f1 * h2f(s1)));
    had128_wave<false>(v0, v1, lane);
    o0 = f2h(v0);
    o1 = f2h(v1);
}

__device__ __forceinline__ uint16_t ldg16(const void* p, int64_t idx) {
    return ((const __attribute__((address_space(1))) uint16_t*)p)[idx];
}

// A staged row's 128-block in LDS, permuted so that each A operand of a step is one ds_read_b128.
__device__ __forceinline__ void lds_put(uint16_t* A, int q, int kp, int col0, int lane, uint16_t v0, uint16_t v1) {
    const int o = perm_slot(lane);
    A[q * kp + col0 + o] = v0;
    A[q * kp + col0 + o + 64] = v1;
}

// prep_gu: one wave per (sorted row i, half m, 128-block b): xr = f16(had128(f16(x * s))) with s = suh (m = 0) or suh1
// (m = 1) of the row's expert. Rows outside every run are not written (include/exl3_abi.h:273-278); a run's row whose
// sorted_tok is negative is written zero.
__global__ __launch_bounds__(256) void k_prep(const Exl3c4Launch a) {
    const int lane = threadIdx.x & 63, el = had_col(lane);
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int nb = a.x_cols_max / 128;
    if (wid >= (int64_t)a.T * 2 * nb) return;
    const int b = (int)(wid % nb);
    const int64_t im = wid / nb;
    const int64_t i = im / 2;
    const int m = (int)(im % 2);
    const int e = owner_wave(a.off, a.n_expert, (int)i, lane);
    if (e < 0) return;
    const int c = class_of(a, e);
    const int64_t jx = entry_of(a, e);
    const Exl3c4DevClass& K = a.cls[c];
    const int C = K.cols;
    if (b * 128 >= C) return;
    uint16_t* out = (uint16_t*)a.y + i * a.y_pitch + (int64_t)m * C + b * 128;
    const int tok = a.sorted[i];
    if (tok < 0) {
        out[lane] = 0;
        out[lane + 64] = 0;
        return;
    }
    int64_t src = tok / a.top_k;
    src = src < a.x_rows ? src : a.x_rows - 1;
    const void* x = (const uint16_t*)a.x + src * a.x_pitch + b * 128;
    const void* s = m ? tab_entry(K.suh1, K.suh1_s, jx) : tab_entry(K.suh, K.suh_s, jx);
    const uint16_t x0 = ldg16(x, el), x1 = ldg16(x, 64 + el);
    const float f0 = a.x_dtype == EXL3C4_BF16 ? bf2f(x0) : h2f(x0);
    const float f1 = a.x_dtype == EXL3C4_BF16 ? bf2f(x1) : h2f(x1);
    uint16_t o0, o1;
    rotate_block(f0, f1, ldg16(s, b * 128 + el), ldg16(s, b * 128 + 64 + el), lane, o0, o1);
    const int et = had_col_t(lane);
    out[et] = o0;
    out[et + 64] = o1;
}

// silu(g) = g / (1 + e^-g) as g x rcp(1 + exp2(-g log2 e)): the hardware exp2 and reciprocal (4 instructions against
// 26 for expf and an IEEE division), within a few f32 ulps of the reference's g * (1 / (1 + expf(-g)))
// (kernels/exl3ref/ref.c:187-212) -- below the f16 rounding of silu(gate) * up that follows, which the reference
// value then meets within one f16 ulp. The same function on every path, so the paths' bits agree.
__device__ __forceinline__ float silu(float g) { return g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }

// A partial sum as gate_up_down's single kernel exchanges it between workgroups: a relaxed atomic access at agent
// scope, coherent across the XCDs' L2 caches by itself (ordered by the row counter: the writer waits for its stores
// before it counts, the reader reads after the count is whole).
template <bool COH> __device__ __forceinline__ float part_ld(const __attribute__((address_space(1))) float* p) {
    if (COH) return __hip_atomic_load((const float*)p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    return *p;
}
template <bool COH> __device__ __forceinline__ void part_st(float* p, float v) {
    if (COH) __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else *p = v;
}

// The split-K partial sums of four columns of sorted row i, added in ascending split order (the order fixes the
// bits). The loads go out R splits at a time (4 R registers): S / R round trips in all. R = min(S, SR), SR the
// caller's budget of registers (4, 8 or 16 splits).
template <bool COH, int R>
__device__ __forceinline__ void sum_rounds(const __attribute__((address_space(1))) float* p, int S, int64_t st,
                                           const int (&col)[4], float (&out)[4]) {
    for (int q0 = 0; q0 < S; q0 += R) {                           // S is a multiple of R (both powers of two)
        float v[4][R];
#pragma unroll
        for (int q = 0; q < R; ++q)
#pragma unroll
            for (int c = 0; c < 4; ++c) v[c][q] = part_ld<COH>(p + (int64_t)(q0 + q) * st + col[c]);
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            float t = q0 == 0 ? v[c][0] : out[c] + v[c][0];
#pragma unroll
            for (int q = 1; q < R; ++q) t = t + v[c][q];
            out[c] = t;
        }
    }
}
template <bool COH, int SR = 4>
__device__ __forceinline__ void sum_splits4(const Exl3c4Launch& a, int64_t i, const int (&col)[4], float (&out)[4]) {
    const __attribute__((address_space(1))) float* p =
        (const __attribute__((address_space(1))) float*)a.part + i * a.part_pitch;
    const int S = a.ksplit;
    const int64_t st = (int64_t)a.T * a.part_pitch;               // one split's sums: [T][part_pitch]
    if (S < 4) {                                                  // 1 or 2
        float v[4][2];
#pragma unroll
        for (int c = 0; c < 4; ++c) {
            v[c][0] = part_ld<COH>(p + col[c]);
            v[c][1] = S == 2 ? part_ld<COH>(p + st + col[c]) : 0.f;
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) out[c] = S == 2 ? v[c][0] + v[c][1] : v[c][0];
        return;
    }
    if (SR >= 16 && S >= 16) sum_rounds<COH, (SR >= 16 ? 16 : 4)>(p, S, st, col, out);
    else if (SR >= 8 && S >= 8) sum_rounds<COH, (SR >= 8 ? 8 : 4)>(p, S, st, col, out);
    else sum_rounds<COH, 4>(p, S, st, col, out);
}

// gate_up's epilogue on one 128-column block of a row, lane l holding gate columns j, j + 64 (acc[0], acc[1]) and up
// columns j, j + 64 (acc[2], acc[3]) of the block's f32 sums (j = had_col(l)), and svh and (h_rot) dn_suh of the
// columns t, t + 64 (t = had_col_t(l)): had128, x svh, f16(silu(gate) * up), and with h_rot down's first step
// f16(had(f16(h * dn_suh))). The result is h's columns t, t + 64 without h_rot, j, j + 64 with it.
__device__ __forceinline__ void gate_up_math(const float (&acc)[4], uint16_t sg0, uint16_t sg1, uint16_t su0,
                                             uint16_t su1, uint16_t d0, uint16_t d1, int h_rot, int lane,
                                             uint16_t& v0, uint16_t& v1) {
    float g0 = acc[0], g1 = acc[1], u0 = acc[2], u1 = acc[3];
    had128_wave<false>(g0, g1, lane);
    had128_wave<false>(u0, u1, lane);
    g0 = g0 * h2f(sg0);
    g1 = g1 * h2f(sg1);
    u0 = u0 * h2f(su0);
    u1 = u1 * h2f(su1);
    const uint16_t h0 = f2h(silu(g0) * u0), h1 = f2h(silu(g1) * u1);
    if (!h_rot) {
        v0 = h0;
        v1 = h1;
        return;
    }
    float r0 = h2f(f2h(h2f(h0) * h2f(d0))), r1 = h2f(f2h(h2f(h1) * h2f(d1)));
    had128_wave<true>(r0, r1, lane);
    v0 = f2h(r0);
    v1 = f2h(r1);
}

// gate_up's output for one 128-column block b of sorted row i (class geometry K, table entry jx), from its partial
// sums: had128, x svh, f16(silu(gate) * up), and with h_rot down's first step f16(had(f16(h * dn_suh))) -- lane l's
// values for columns b * 128 + (h_rot ? had_col(l) : had_col_t(l)) (v0) and + 64 (v1), as fp16 bits (docs/OPS-exl3.md:104-123; kernels/exl3ref/ref.c:
// 187-212).
template <bool COH, int SR = 4>
__device__ __forceinline__ void gate_up_block(const Exl3c4Launch& a, const Exl3c4DevClass& K, int64_t i, int b,
                                              int64_t jx, int h_rot, int lane, uint16_t& v0, uint16_t& v1) {
    const void* svh = tab_entry(K.svh, K.svh_s, jx);
    const int n0 = b * 128 + had_col(lane), n1 = n0 + 64;        // the sums' columns
    const int t0 = b * 128 + had_col_t(lane), t1 = t0 + 64;      // the scales' columns
    const int width = K.rows / 2;
    const uint16_t sg0 = ldg16(svh, t0), sg1 = ldg16(svh, t1), su0 = ldg16(svh, width + t0), su1 = ldg16(svh, width + t1);
    const void* ds = h_rot ? tab_entry(K.dn_suh, K.dn_suh_s, jx) : nullptr;
    const uint16_t d0 = h_rot ? ldg16(ds, t0) : 0, d1 = h_rot ? ldg16(ds, t1) : 0;
    const int col[4] = { n0, n1, width + n0, width + n1 };
    float acc[4];
    sum_splits4<COH, SR>(a, i, col, acc);
    gate_up_math(acc, sg0, sg1, su0, su1, d0, d1, h_rot, lane, v0, v1);
}

typedef const uint32_t __attribute__((address_space(1)))* gu32p;

// One step of the decode GEMV: the wave's segment decoded into B operands and the four MFMAs against the staged rows
// (arow: this lane's row and k group in LDS).
template <int BITS, int CB>
__device__ __forceinline__ void mma_step(const uint32_t (&d)[BITS], const uint16_t* arow, const Mul1Consts& k,
                                         float4_t& acc0, float4_t& acc1) {
    uint32_t B[16];
    decode_segment<BITS, CB>(d, B, k);
    const half8_t Aa = *(const half8_t*)(arow);
    const half8_t Ab = *(const half8_t*)(arow + 8);
    const half8_t b0 = as_half8(B[0], B[1], B[2], B[3]), b1 = as_half8(B[8], B[9], B[10], B[11]);
    const half8_t b2 = as_half8(B[4], B[5], B[6], B[7]), b3 = as_half8(B[12], B[13], B[14], B[15]);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Aa, b0, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Aa, b1, acc1, 0, 0, 0);
    acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ab, b2, acc0, 0, 0, 0);
    acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ab, b3, acc1, 0, 0, 0);
    mfma_guard(Aa, Ab, b0, b1, b2, b3);
}

// The codes of the next PF steps of a wave's stream: in flight while the earlier steps are decoded.
#ifndef EXL3C4_GEMV_PF
#define EXL3C4_GEMV_PF 2
#endif
template <int BITS> struct CodeRing { uint32_t d[EXL3C4_GEMV_PF][BITS]; };

template <int BITS> __device__ __forceinline__ void prime(gu32p rec, int ksn, CodeRing<BITS>& r) {
#pragma unroll
    for (int q = 0; q < EXL3C4_GEMV_PF; ++q)
        if (q < ksn) load_words<BITS>(rec + q * 64 * BITS, r.d[q]);
}

// The wave's strip over `ksn` steps of its stream `rec`, whose first steps' words are already in flight in `r`
// (prime), against the rows staged in LDS.
template <int BITS, int CB>
__device__ __forceinline__ void gemv_strip(gu32p rec, int ksn, CodeRing<BITS>& r, const uint16_t* arow,
                                           float4_t& acc0, float4_t& acc1) {
    const Mul1Consts k = mul1_consts();
    constexpr int PF = EXL3C4_GEMV_PF;
    // ksn is even (two steps a 128-block), so with PF two both steps of a pair exist; a deeper ring ends the stream
    // with a partial round. The refill is unconditional (past the stream a harmless reload of the last step), so the
    // waits for the codes are counted, not drained.
    static_assert(PF >= 2 && PF <= 4, "gemv_strip keeps two to four steps in flight");
    for (int s = 0; s < ksn; s += PF) {
#pragma unroll
        for (int q = 0; q < PF; ++q) {
            if (PF > 2 && s + q >= ksn) break;
            mma_step<BITS, CB>(r.d[q], arow + (s + q) * EXL3C4_KSTEP, k, acc0, acc1);
            const int nx = s + q + PF < ksn ? s + q + PF : ksn - 1;
            load_words<BITS>(rec + nx * 64 * BITS, r.d[q]);
        }
    }
}

// gate_up's staging of a split's input rows in LDS (the split's 128-blocks [b0, b1)): as given (AROT: x holds the
// rotated rows, the gate half then the up half) or f16(had128(f16(x * s))) of the row's token (s = suh or suh1, zero
// for a negative sorted_tok). The (row, block) pairs of the chunk, row-major, are dealt to the four waves, PB a wave
// a round: a round's input and scale loads all go out before any is used, none behind a branch (a pair past the last
// loads the last, unused), so a round costs one memory round trip however its pairs fall over rows and blocks (a chunk
// of 16 rows and one block: one round, not 16 round trips in series). The codes' first steps go out right after the
// first round's inputs, so they are in flight while it is staged; the codes are not waited for before the loop.
// A chunk of at most four pairs (the decode layer's one-row chunks: a split's four blocks) takes one round of one pair
// a wave, without the loads and addresses of three unused pairs a wave.
template <int BITS, bool AROT, int PB>
__device__ __forceinline__ void gu_stage_rounds(const Exl3c4Launch& a, int i, int npair, int nbs, int KC, bool up,
                                                int b0, int tok_l, const void* sv, gu32p rec, int ksn,
                                                CodeRing<BITS>& ring, uint16_t* A, int kp) {
    const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 6), lane = threadIdx.x & 63, el = had_col(lane);
    const int eo = AROT ? el : had_col_t(lane);                   // where a staged value goes
    const bool bf = a.x_dtype == EXL3C4_BF16;
    for (int p0 = 0; p0 < npair; p0 += 4 * PB) {
        int q[PB], hb[PB], tok[PB];
        uint16_t x0[PB], x1[PB], s0[PB], s1[PB];
#pragma unroll
        for (int j = 0; j < PB; ++j) {                            // wave-uniform: the pair's row and block
            const int pc = min(p0 + wave + 4 * j, npair - 1);
            q[j] = pc / nbs;
            hb[j] = b0 + (pc - q[j] * nbs);
            tok[j] = AROT ? 0 : __builtin_amdgcn_readlane(tok_l, q[j]);
            int64_t src = AROT ? (int64_t)i + q[j] : (tok[j] >= 0 ? tok[j] / a.top_k : 0);
            src = src < a.x_rows ? src : a.x_rows - 1;
            const uint16_t* xr = (const uint16_t*)a.x + src * a.x_pitch + (AROT && up ? KC : 0);
            x0[j] = ldg16(xr, hb[j] * 128 + el);
            x1[j] = ldg16(xr, hb[j] * 128 + 64 + el);
        }
        if (p0 == 0) prime<BITS>(rec, ksn, ring);
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            s0[j] = AROT ? 0 : ldg16(sv, hb[j] * 128 + el);
            s1[j] = AROT ? 0 : ldg16(sv, hb[j] * 128 + 64 + el);
        }
#pragma unroll
        for (int j = 0; j < PB; ++j) {
            if (p0 + wave + 4 * j >= npair) break;                // uniform: the rotation's DPP runs the whole wave
            uint16_t v0 = x0[j], v1 = x1[j];
            if (!AROT) {
                v0 = v1 = 0;
                if (tok[j] >= 0)
                    rotate_block(bf ? bf2f(x0[j]) : h2f(x0[j]), bf ? bf2f(x1[j]) : h2f(x1[j]), s0[j], s1[j], lane, v0,
                                 v1);
            }
            lds_put(A, q[j], kp, (hb[j] - b0) * 128, eo, v0, v1);
        }
    }
}
template <int BITS, bool AROT>
__device__ __forceinline__ void gu_stage(const Exl3c4Launch& a, int i, int nrows, int KC, bool up, int b0, int b1,
                                         int tok_l, const void* sv, gu32p rec, int ksn, CodeRing<BITS>& ring,
                                         uint16_t* A, int kp) {
    const int nbs = b1 - b0, npair = nrows * nbs;
    if (npair <= 4) gu_stage_rounds<BITS, AROT, 1>(a, i, npair, nbs, KC, up, b0, tok_l, sv, rec, ksn, ring, A, kp);
    else gu_stage_rounds<BITS, AROT, 4>(a, i, npair, nbs, KC, up, b0, tok_l, sv, rec, ksn, ring, A, kp);
}

// gate_up's GEMM: one workgroup per (sorted row i, group of four 32-column strips, k split). The workgroup keyed on
// a chunk's first row takes the chunk (at most 16 rows); the others leave. Its four waves take the group's four
// strips over the split's 128-blocks of k; the split's input rows -- rotated here, f16(had128(f16(x * suh or suh1)))
// of the token's row, or read as given (a_rot) -- are staged once in LDS for all four. The strip's sums go to
// part[split][row][col]; their consumer adds the splits in a fixed order, so the bits do not depend on scheduling.
// Unit u = group u >> ksplit_log2, split u & (S - 1) of row i; kp: halves a staged row. Returns the chunk's rows (0 when
// row i starts none) and the row's owner. In its own kernel (k_gu) unit 0 of each row records the row's owner and chunk rows in row_info
// for the kernels that follow; inside gate_up_down's single launch (FUSED) nothing follows, so it records nothing.
struct GuRows { int nrows, e; };
template <int BITS, int CB, bool FUSED>
__device__ __forceinline__ GuRows gu_unit(const Exl3c4Launch& a, int i, int u, int kp, unsigned char* lds) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int S = a.ksplit;
    const int grp = u >> a.ksplit_log2, split = u & (S - 1);
    // the chunk's sorted_tok (lane q: row i + q), read beside the owner search (taken by readlane below)
    const int tok_l = a.sorted[min(i + (lane & 15), a.T - 1)];
    const Owner w = owner_wg(a, i);
    const int nrows = chunk_rows(a, w, i);
    if (!FUSED && u == 0 && threadIdx.x == 0) {
        a.row_info[2 * i] = w.e;
        a.row_info[2 * i + 1] = nrows;
    }
    if (nrows == 0) return GuRows{ 0, w.e };
    const int c = class_of(a, w.e);
    const int64_t jx = entry_of(a, w.e);
    const Exl3c4DevClass& K = a.cls[c];
    const int N = K.rows, KC = K.cols;
    if (grp * 128 >= N) return GuRows{ nrows, w.e };
    const int strip = grp * 4 + wave;
    const bool up = grp * 128 >= N / 2;
    const int nb = KC / 128, per = (nb + S - 1) / S;
    const int b0 = min(nb, split * per), b1 = min(nb, b0 + per);
    const int ksn = 2 * (b1 - b0);
    const gu32p rec = (gu32p)tab_entry(K.codes, K.codes_s, jx) +
                      ((int64_t)strip * (KC / EXL3C4_KSTEP) + 2 * b0) * 64 * BITS + lane * BITS;
    CodeRing<BITS> ring;

    uint16_t* A = (uint16_t*)lds;                                 // [chunk_rows][kp]
    if (ksn > 0) {
        if (a.a_rot) gu_stage<BITS, true>(a, i, nrows, KC, up, b0, b1, tok_l, nullptr, rec, ksn, ring, A, kp);
        else gu_stage<BITS, false>(a, i, nrows, KC, up, b0, b1, tok_l,
                                   up ? tab_entry(K.suh1, K.suh1_s, jx) : tab_entry(K.suh, K.suh_s, jx), rec, ksn,
                                   ring, A, kp);
    }
    __syncthreads();

    float4_t acc0 = { 0.f, 0.f, 0.f, 0.f }, acc1 = { 0.f, 0.f, 0.f, 0.f };
    gemv_strip<BITS, CB>(rec, ksn, ring, A + a_row(a, lane) * kp + 16 * (lane >> 4), acc0, acc1);

    // D lane l: column l % 16 (c' = 2 s + t -> weight row 32 nb + 16 t + s, + 8 for acc1), rows 4 (l / 16) + 0..3
    const int cc = lane & 15, rg = lane >> 4;
    const int n = strip * EXL3C4_STRIP + 16 * (cc & 1) + (cc >> 1);
    float* pp = a.part + (int64_t)split * a.T * a.part_pitch;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int tok = rg * 4 + q;
        if (tok < nrows) {
            part_st<FUSED>(pp + (int64_t)(i + tok) * a.part_pitch + n, acc0[q]);
            part_st<FUSED>(pp + (int64_t)(i + tok) * a.part_pitch + n + 8, acc1[q]);
        }
    }
    return GuRows{ nrows, w.e };
}

template <int BITS, int CB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(6, 8))) void k_gu(const Exl3c4Launch a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    gu_unit<BITS, CB, false>(a, blockIdx.y, blockIdx.x, a.lds_pitch, lds);
}

// gate_up's epilogue (gate_up alone): one wave per (sorted row i, 128-column block b) of h, from the partial sums.
// A row no run holds, a negative sorted_tok and a narrower class's tail are written zero.
// SR: split-K sums loaded a round (8 for S >= 8, the launches of few rows: one round trip where S = 16 took four).
template <int SR>
__global__ __launch_bounds__(256) void k_gepi(const Exl3c4Launch a) {
    const int lane = threadIdx.x & 63, el = a.h_rot ? had_col(lane) : had_col_t(lane);  // h's columns
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int per = max(1, a.blk_per_wave), nw = (a.nblk + per - 1) / per;   // a wave takes `per` blocks of a row
    if (wid >= (int64_t)a.T * nw) return;
    const int64_t i = wid / nw;
    const int b0 = (int)(wid % nw) * per, b1 = min(a.nblk, b0 + per);
    const int e = a.row_info[2 * i];
    const int c = e >= 0 ? class_of(a, e) : 0;
    const bool dead = e < 0 || a.sorted[i] < 0;
    for (int b = b0; b < b1; ++b) {
        uint16_t* out = (uint16_t*)a.y + i * a.y_pitch + b * 128;
        uint16_t v0 = 0, v1 = 0;
        if (!dead && b * 128 < a.cls[c].rows / 2)
            gate_up_block<false, SR>(a, a.cls[c], i, b, entry_of(a, e), a.h_rot, lane, v0, v1);
        out[el] = v0;
        out[el + 64] = v1;
    }
}

// Row i's counter: each in its own cache line, so that polls and counts of different rows do not meet. Half a line on,
// EXL3C4_SYNC_DONE words in, the count of the row's down units past their wait.
__device__ __forceinline__ int32_t* row_counter(const Exl3c4Launch& a, int i) {
    return a.sync + (int64_t)(i + 1) * EXL3C4_SYNC_STRIDE;
}

// A down unit of gate_up_down's single launch waits here until its chunk's h is stored: row i's counter reaches
// n_grp x ksplit + 1 (one count per gate_up unit of row i once its sums are stored, one more once the last of them has
// formed h). The wait gives up after EXL3C4_WAIT_TICKS of the 100 MHz clock, or soon after another workgroup gave up,
// and sets bit 0 of the status word sync[0] -- and *fail, a flag the host can read without a synchronisation, when
// the launch has one (the plugin rows' instances) -- the output is then void; the launch still ends.
// A status word already set when the wait begins also gives up at once, before any counter is read: a block whose
// earlier launch gave up may hold stale counts (a late gate_up count lands after the row's down units zeroed the
// row's counters), so every later launch on it is void and reports it again -- in the same launch -- until the
// caller zeroes the block.
#define EXL3C4_WAIT_TICKS 50000000ull
__device__ __forceinline__ void wait_gate_up(const Exl3c4Launch& a, int i) {
    if (threadIdx.x == 0) {
        const int want = (a.n_grp << a.ksplit_log2) + 1;
        const int32_t* cnt = row_counter(a, i);
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        // the status word and the first poll go out together: no round trip more on the wait's path
        const int32_t st = __hip_atomic_load(a.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        int32_t c = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        bool give_up = (st & 1) != 0;
        for (unsigned n = 1; !give_up && c < want; ++n) {
            __builtin_amdgcn_s_sleep(8);
            give_up = (n & 15) == 0 && ((__hip_atomic_load(a.sync, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) & 1) ||
                                        __builtin_amdgcn_s_memrealtime() - t0 > EXL3C4_WAIT_TICKS);
            c = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (give_up) {
            __hip_atomic_fetch_or(a.sync, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (a.fail) __hip_atomic_store(a.fail, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        }
    }
    __syncthreads();
}

// down, one workgroup per (sorted row i, 128-column output block b); the workgroup keyed on a chunk's first row takes
// the chunk. Its four waves take the block's four 32-column strips over all of k, so the block's output is whole
// inside the workgroup and its epilogue (had128, x svh, bf16) runs there. The chunk's input rows are staged in LDS
// first: gate_up's h_rot = 1 output computed from gate_up's partial sums (gate_up_down), or the rows of x, rotated
// (h_rot = 0) or as given (down alone). The raw accumulations also go to `dacc` (a checker's view of the sums before
// any narrowing). Every (row, block) of y is written once: a row no run holds, a negative sorted_tok and a narrower
// class's tail as zero. Inside gate_up_down's single launch (FUSED) the workgroup finds the row's owner itself and
// waits for the row's gate_up units before it reads their sums.
// y's 128-block b of one row: coherent stores when the launch gathers (the gathering unit may sit on another XCD and
// reads them with coherent loads once every unit of the token's rows has counted, after its stores completed)
__device__ __forceinline__ void put_y(const Exl3c4Launch& a, uint16_t* out, int lane, uint16_t v0, uint16_t v1) {
    if (a.g_out) {
        __hip_atomic_store(out + lane, v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(out + lane + 64, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    } else {
        out[lane] = v0;
        out[lane + 64] = v1;
    }
}

// moe_gather behind gate_up_down's single launch (g_out set): a down unit that has stored its chunk's rows of block b
// counts each live row on its token's counter of block b; the count that completes a token (its slots with a row,
// from row_of) gathers that token's block -- k_gather's sum: the slots in ascending order, one f32 product and one add
// each, f16 -- over the rows' y read coherently, then sets the counter back to zero. No unit waits here. A chunk holds
// a token at most once (its slots name distinct experts), at most 16 rows at decode. Wave w takes rows w, w + 4, ..:
// the row's count and its token's first 16 slots (rows and weights, lane u slot u) go out together, so a completing
// count finds the slots in registers and the gather's first loads are the rows' y.
__device__ void gather_count(const Exl3c4Launch& a, int i, int nrows, int b, int tok_l) {
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");              // this thread's y stores are done
    __syncthreads();                                              // ... and the workgroup's: the counts may go out
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int K = a.top_k;
    for (int q = wave; q < nrows; q += 4) {                       // k_gd: 4 waves a workgroup
        const int p = __builtin_amdgcn_readlane(tok_l, q);        // tok_l: sorted_tok of row i + lane
        const int64_t t = p >= 0 ? p / K : -1;
        if (t < 0 || t >= a.g_ntok) continue;
        int old = 0;
        if (lane == 0)
            old = __hip_atomic_fetch_add(a.g_ctr + t * EXL3C4_SYNC_STRIDE + b, 1, __ATOMIC_RELAXED,
                                         __HIP_MEMORY_SCOPE_AGENT);
        // the token's slots with a row (0 <= row < T, as the sum and gather_empty read it), read while the count is
        // in flight (clamped addresses, none behind a branch)
        const int sl_l = min(lane & 15, K - 1);
        const int r_first = a.g_row_of[t * K + sl_l];
        const float w_first = a.g_w[t * K + sl_l];
        int need = __popcll(__ballot(lane < 16 && lane < K && r_first >= 0 && r_first < a.T));
        for (int s0 = 16; s0 < K; s0 += 64) {
            const int r = a.g_row_of[t * K + min(s0 + lane, K - 1)];
            need += __popcll(__ballot(s0 + lane < K && r >= 0 && r < a.T));
        }
        if (__builtin_amdgcn_readlane(old, 0) != need - 1) continue;
        const int c = b * 128 + lane;
        float acc0 = 0.f, acc1 = 0.f;
        for (int s0 = 0; s0 < K; s0 += 16) {                      // 16 slots' rows and weights, then their values
            // lane u holds slot s0 + u (the first 16 from the count's loads), each then taken uniform by readlane
            int r_l = r_first;
            float w_l = w_first;
            if (s0 > 0) {
                const int sl = min(s0 + (lane & 15), K - 1);
                r_l = a.g_row_of[t * K + sl];
                w_l = a.g_w[t * K + sl];
            }
            int r[16];
            float w[16];
            uint16_t q0[16], q1[16];
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                r[u] = __builtin_amdgcn_readlane(r_l, u);
                w[u] = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(w_l), u));
                if (s0 + u >= a.top_k || r[u] >= a.T) r[u] = -1;
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const uint16_t* yr = (const uint16_t*)a.y + (int64_t)(r[u] < 0 ? 0 : r[u]) * a.y_pitch + c;
                q0[u] = __hip_atomic_load(yr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                q1[u] = __hip_atomic_load(yr + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
#pragma unroll
            for (int u = 0; u < 16; ++u) {
                const float p0 = w[u] * bf2f(q0[u]), p1 = w[u] * bf2f(q1[u]);
                const float s0v = acc0 + p0, s1v = acc1 + p1;
                acc0 = r[u] < 0 ? acc0 : s0v;                     // a pair without a row adds nothing
                acc1 = r[u] < 0 ? acc1 : s1v;
            }
        }
        uint16_t* o = a.g_out + t * a.g_out_pitch + c;
        o[0] = f2h(acc0);
        o[64] = f2h(acc1);
        if (lane == 0)
            __hip_atomic_store(a.g_ctr + t * EXL3C4_SYNC_STRIDE + b, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

// The gather's tokens with no slot holding a row (no unit counts them): out zero, as k_gather writes. Wave w of job z
// takes token 4 z + w.
__device__ __forceinline__ void gather_empty(const Exl3c4Launch& a, int z) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)z * 4 + (threadIdx.x >> 6);        // k_gd: 4 waves a workgroup
    if (t >= a.g_ntok) return;
    for (int s0 = 0; s0 < a.top_k; s0 += 64) {                    // lane u reads slot s0 + u
        const int r = a.g_row_of[t * a.top_k + min(s0 + lane, a.top_k - 1)];
        if (__ballot(s0 + lane < a.top_k && r >= 0 && r < a.T)) return;
    }
    for (int c = lane; c < a.y_cols; c += 64) a.g_out[t * a.g_out_pitch + c] = 0;
}

// down's weight as a kernel reads it: the op's own (the down op), or gate_up_down's -- dn_codes / dn_svh of gate_up's
// class, [cols, rows / 2], with suh = dn_suh (include/exl3_abi.h:751-800)
struct DnW { const void *codes, *svh, *suh; int32_t codes_s, svh_s, suh_s; int rows, cols; };
__device__ __forceinline__ DnW dn_weight(bool gd, const Exl3c4DevClass& K) {
    if (gd) return DnW{ K.dn_codes, K.dn_svh, K.dn_suh, K.dn_codes_s, K.dn_svh_s, K.dn_suh_s, K.cols, K.rows / 2 };
    return DnW{ K.codes, K.svh, K.suh, K.codes_s, K.svh_s, K.suh_s, K.rows, K.cols };
}

// Down's staging of h inside gate_up_down's single launch: wave w stages h's block w of the chunk's rows (at most R),
// every row's loads first, none behind a branch (rows past the chunk's last and blocks past h's last load those,
// unused); R the least of 1, 4, 8, 16 that holds the chunk, so a one-row chunk issues two loads a lane, not 32.
template <int R>
__device__ __forceinline__ void dn_stage_h(const Exl3c4Launch& a, int i, int nrows, int nhb, int wave, int lane,
                                           uint16_t* A, int kp) {
    const int hb = wave;
    uint16_t h0[R], h1[R];
#pragma unroll
    for (int q = 0; q < R; ++q) {
        const uint16_t* hs = a.hbuf + (int64_t)(i + min(q, nrows - 1)) * a.hbuf_pitch + min(hb, nhb - 1) * 128;
        h0[q] = __hip_atomic_load(hs + lane, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        h1[q] = __hip_atomic_load(hs + lane + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int q = 0; q < R; ++q)
        if (q < nrows && hb < nhb) lds_put(A, q, kp, hb * 128, lane, h0[q], h1[q]);
}

template <int BITS, int CB, bool FUSED>
__device__ __forceinline__ void dn_unit(const Exl3c4Launch& a, int b, int i, unsigned char* lds) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    // the chunk's sorted_tok (lane q: row i + q), read beside the owner search: the epilogue and the gather take it
    const int tok_l = a.sorted[min(i + (lane & 15), a.T - 1)];
    int e, nrows;
    if (!FUSED && a.row_info) {                                   // uniform: the class tables by scalar loads
        e = __builtin_amdgcn_readfirstlane(a.row_info[2 * i]);
        nrows = __builtin_amdgcn_readfirstlane(a.row_info[2 * i + 1]);
    } else {
        const Owner w = owner_wg(a, i);
        e = w.e;
        nrows = chunk_rows(a, w, i);
    }
    if (e < 0) {
        if (wave == 0) {
            uint16_t* out = (uint16_t*)a.y + (int64_t)i * a.y_pitch + b * 128;
            out[lane] = 0;
            out[lane + 64] = 0;
        }
        return;
    }
    if (nrows == 0) return;
    const int c = class_of(a, e);
    const int64_t jx = entry_of(a, e);
    const DnW D = dn_weight(FUSED || a.dn_gd, a.cls[c]);
    const int N = D.rows, KC = D.cols;
    if (b * 128 >= N) {                                           // a narrower class's tail
        for (int q = wave; q < nrows; q += 4)
            put_y(a, (uint16_t*)a.y + (int64_t)(i + q) * a.y_pitch + b * 128, lane, 0, 0);
        if (FUSED && a.g_out) gather_count(a, i, nrows, b, tok_l);
        return;
    }
    const int kp = a.lds_pitch;               // halves a staged row: k plus 8, so the 16 rows fall in different banks
    uint16_t* A = (uint16_t*)lds;                                 // [chunk_rows][kp]
    float* acc_l = (float*)lds;                                   // [chunk_rows][128], over A once the waves are done

    // this wave's strip of the block, all of k; its first codes are in flight while the rows are staged
    const int strip = 4 * b + wave;
    const int ksteps = KC / EXL3C4_KSTEP;
    const gu32p rec = (gu32p)tab_entry(D.codes, D.codes_s, jx) + (int64_t)strip * ksteps * 64 * BITS + lane * BITS;
    CodeRing<BITS> ring;
    prime<BITS>(rec, ksteps, ring);
    const void* svh = tab_entry(D.svh, D.svh_s, jx);
    const int el = had_col(lane), et = had_col_t(lane);          // the block's sums' columns, its outputs'
    const uint16_t sv0 = ldg16(svh, b * 128 + et), sv1 = ldg16(svh, b * 128 + 64 + et);
    const void* suh = (!a.h_from_gu && !a.h_rot) ? tab_entry(D.suh, D.suh_s, jx) : nullptr;
    if (FUSED) wait_gate_up(a, i);
    // every down unit of the row has passed its wait once the row's last one counts here: that one zeroes the row's
    // counters at its end, so a launch leaves them as it found them (the reference's counter blocks,
    // kernels/exl3r4d/launch.c:311-324). Counted right after the wait, so the count's round trip runs under the
    // staging and the loop rather than at the unit's end.
    int done_old = 0;
    if (FUSED && threadIdx.x == 0)
        done_old = __hip_atomic_fetch_add(row_counter(a, i) + EXL3C4_SYNC_DONE, 1, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT);

    // stage the chunk's rows
    const int nhb = KC / 128;
    if (FUSED && nhb <= 4) {                                      // each wave one block of h (dn_stage_h)
        if (nrows <= 1) dn_stage_h<1>(a, i, nrows, nhb, wave, lane, A, kp);
        else if (nrows <= 4) dn_stage_h<4>(a, i, nrows, nhb, wave, lane, A, kp);
        else if (nrows <= 8) dn_stage_h<8>(a, i, nrows, nhb, wave, lane, A, kp);
        else dn_stage_h<EXL3C4_CHUNK_ROWS>(a, i, nrows, nhb, wave, lane, A, kp);
    } else if (!FUSED && !a.h_from_gu) {                          // down's input rows (its op's, or h from k_gepi):
        // each of a wave's blocks with every row's loads first, none behind a branch (rows past the chunk load its
        // last, unused): a block costs one round trip, not one a row
        for (int hb = wave; hb < nhb; hb += 4) {                  // uniform in the wave
            if (a.h_rot) {                                        // as given: columns 2 l, 2 l + 1 a lane, one dword
                constexpr int R = EXL3C4_CHUNK_ROWS;              // (they are adjacent in the permuted layout too)
                uint32_t h[R];
#pragma unroll
                for (int q = 0; q < R; ++q) {
                    const uint16_t* xs = (const uint16_t*)a.x + (int64_t)(i + min(q, nrows - 1)) * a.x_pitch + hb * 128;
                    h[q] = *(const __attribute__((address_space(1))) uint32_t*)(xs + 2 * lane);
                }
                const int o = perm_slot(2 * lane);
#pragma unroll
                for (int q = 0; q < R; ++q)
                    if (q < nrows) *(uint32_t*)(A + q * kp + hb * 128 + o) = h[q];
            } else {                                              // rotated here: f16(had128(f16(x * suh)))
                constexpr int R = EXL3C4_CHUNK_ROWS / 2;          // eight rows' loads at a time
                const uint16_t s0 = ldg16(suh, hb * 128 + el), s1 = ldg16(suh, hb * 128 + 64 + el);
                for (int q0 = 0; q0 < nrows; q0 += R) {
                    uint16_t h0[R], h1[R];
#pragma unroll
                    for (int q = 0; q < R; ++q) {
                        const uint16_t* xs =
                            (const uint16_t*)a.x + (int64_t)(i + min(q0 + q, nrows - 1)) * a.x_pitch + hb * 128;
                        h0[q] = ldg16(xs, el);
                        h1[q] = ldg16(xs, el + 64);
                    }
#pragma unroll
                    for (int q = 0; q < R; ++q) {
                        if (q0 + q < nrows) {                     // uniform: the rotation's DPP runs the whole wave
                            uint16_t v0, v1;
                            rotate_block(h2f(h0[q]), h2f(h1[q]), s0, s1, lane, v0, v1);
                            lds_put(A, q0 + q, kp, hb * 128, et, v0, v1);
                        }
                    }
                }
            }
        }
    } else for (int q = 0; q < nrows; ++q) {
        const int64_t r = i + q;
        for (int hb = wave; hb < nhb; hb += 4) {
            uint16_t v0 = 0, v1 = 0;
            int ep = el;                                          // where the staged values go
            if (FUSED) {                                          // the row's h, formed once (row_h)
                const uint16_t* hs = a.hbuf + r * a.hbuf_pitch + hb * 128;
                v0 = __hip_atomic_load(hs + el, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                v1 = __hip_atomic_load(hs + el + 64, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else if (a.h_from_gu) {
                if (a.sorted[r] >= 0) gate_up_block<false>(a, a.cls[c], r, hb, jx, 1, lane, v0, v1);
            } else {
                const void* xs = (const uint16_t*)a.x + r * a.x_pitch + hb * 128;
                const uint16_t x0 = ldg16(xs, el), x1 = ldg16(xs, el + 64);
                if (a.h_rot) {
                    v0 = x0;
                    v1 = x1;
                } else {
                    rotate_block(h2f(x0), h2f(x1), ldg16(suh, hb * 128 + el), ldg16(suh, hb * 128 + 64 + el), lane,
                                 v0, v1);
                    ep = et;
                }
            }
            lds_put(A, q, kp, hb * 128, ep, v0, v1);
        }
    }
    __syncthreads();

    float4_t acc0 = { 0.f, 0.f, 0.f, 0.f }, acc1 = { 0.f, 0.f, 0.f, 0.f };
    gemv_strip<BITS, CB>(rec, ksteps, ring, A + a_row(a, lane) * kp + 16 * (lane >> 4), acc0, acc1);

    // the block's accumulations to LDS (column of D lane l: 16 (l & 1) + (l / 2) within the strip, + 8 for acc1)
    __syncthreads();
    const int cc = lane & 15, rg = lane >> 4;
    const int col = 32 * wave + 16 * (cc & 1) + (cc >> 1);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int tok = rg * 4 + q;
        if (tok < nrows) {
            acc_l[tok * 128 + col] = acc0[q];
            acc_l[tok * 128 + col + 8] = acc1[q];
        }
    }
    __syncthreads();

    for (int q = wave; q < nrows; q += 4) {
        const int64_t r = i + q;
        float y0 = acc_l[q * 128 + el], y1 = acc_l[q * 128 + el + 64];
        float* dacc = a.dacc + r * a.dacc_pitch + b * 128;
        dacc[el] = y0;
        dacc[el + 64] = y1;
        uint16_t* out = (uint16_t*)a.y + r * a.y_pitch + b * 128;
        if (__builtin_amdgcn_readlane(tok_l, q) < 0) {
            put_y(a, out, el, 0, 0);
            continue;
        }
        had128_wave<false>(y0, y1, lane);
        const uint32_t yb = f2bf2(y0 * h2f(sv0), y1 * h2f(sv1));
        put_y(a, out, et, (uint16_t)yb, (uint16_t)(yb >> 16));
    }
    if (FUSED && a.g_out) gather_count(a, i, nrows, b, tok_l);
    if (FUSED && threadIdx.x == 0 && done_old == N / 128 - 1) {
        __hip_atomic_store(row_counter(a, i), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(row_counter(a, i) + EXL3C4_SYNC_DONE, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
}

template <int BITS, int CB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(5, 8))) void k_dn(const Exl3c4Launch a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    dn_unit<BITS, CB, false>(a, blockIdx.x, blockIdx.y, lds);
}

// h of a chunk's rows (gate_up's epilogue with h_rot: had128, x svh, f16(silu(gate) * up), f16(had(f16(h * dn_suh))))
// from the rows' partial sums, once, by the row's last gate_up unit: into hbuf, then one more count on row i's counter.
__device__ __forceinline__ void row_h(const Exl3c4Launch& a, int i, const GuRows& g) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, el = had_col(lane);
    const int c = class_of(a, g.e);
    const int64_t jx = entry_of(a, g.e);
    const Exl3c4DevClass& G = a.cls[c];
    const int nhb = G.rows / 256;                                  // h's 128-blocks: (rows / 2) / 128
    for (int t = wave; t < g.nrows * nhb; t += 4) {
        const int q = t / nhb, hb = t - q * nhb;
        const int64_t r = i + q;
        uint16_t v0, v1;                                          // the row's loads and sorted_tok's together
        gate_up_block<true>(a, G, r, hb, jx, 1, lane, v0, v1);
        if (a.sorted[r] < 0) v0 = v1 = 0;
        uint16_t* h = a.hbuf + r * a.hbuf_pitch + hb * 128;
        __hip_atomic_store(h + el, v0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        __hip_atomic_store(h + el + 64, v1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (threadIdx.x == 0) __hip_atomic_fetch_add(row_counter(a, i), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// gate_up_down in one launch (decode path). Workgroups g = 8 k + x (x < 8) take the sorted rows i = x (mod 8): first
// every gate_up unit of those rows (row-major, the n_grp x ksplit units of k_gu), then every down unit (row-major, the
// nblk blocks of k_dn). A gate_up unit of a chunk's row adds one to its counter once its sums are stored, and the last of
// them forms the chunk's h (row_h) and adds one more; a down unit of that row waits for n_grp x ksplit + 1. The dispatcher deals workgroups to the 8 XCDs in turn and each XCD starts its
// workgroups in order, so the workgroups g = x (mod 8) share one XCD (its L2 holds the row's sums) and when a down unit
// runs, every gate_up unit before it has started; gate_up units never wait, so the waits end. The sums cross as
// coherent accesses (part_ld / part_st), so the bits do not depend on where a workgroup lands. Built for 7 workgroups
// a CU up to K = 6 (the register count it holds either way at K = 4; the schedule this target gives measured 0.5 us
// faster); K = 7, 8 keep the looser target, under which they need no spill.
template <int BITS, int CB, int BD = BITS>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu((BITS > BD ? BITS : BD) <= 6 ? 7 : 5, 8))) void k_gd(
    const Exl3c4Launch a) {
    extern __shared__ __attribute__((aligned(16))) unsigned char lds[];
    const int xcd = (int)(blockIdx.x & 7), slot = (int)(blockIdx.x >> 3);
    const int rows = xcd < a.T ? (a.T - 1 - xcd) / 8 + 1 : 0;
    const int ugu = a.n_grp << a.ksplit_log2;
    if (slot < rows * ugu) {
        const int i = xcd + 8 * (slot / ugu);
        const GuRows g = gu_unit<BITS, CB, true>(a, i, slot % ugu, a.lds_pitch_gu, lds);   // gate_up at K = BITS
        if (g.nrows > 0) {
            __shared__ int last_s;
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");          // this thread's sums are stored
            __syncthreads();
            if (threadIdx.x == 0)
                last_s = __hip_atomic_fetch_add(row_counter(a, i), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
                         ugu - 1;
            __syncthreads();
            if (last_s) row_h(a, i, g);                                // the row's last gate_up unit forms h
        }
        return;
    }
    const int d = slot - rows * ugu;
    if (d < rows * a.nblk) dn_unit<BD, CB, true>(a, d % a.nblk, xcd + 8 * (d / a.nblk), lds);     // down at K = BD
    else if (a.g_out) gather_empty(a, 8 * (d - rows * a.nblk) + xcd);  // the grid's last slots of each XCD
}

__global__ __launch_bounds__(256) void k_fill(int32_t* p, int64_t n) {
    const int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (j < n) p[j] = 0;
}

// ------------------------------------------------------------------------------------------------ the prefill path
//
// Many rows an expert: each weight is decoded once per chunk of up to 64 rows of its run and fed to 4 row tiles of
// MFMAs. The launches: a plan (the chunks, and each row's owner), the input rotation into scratch (xr, as prep_gu
// writes it, or down's rotated h), the GEMMs, and the epilogues.

// One workgroup: every expert's run clamped to [0, T) cut into chunks of at most 64 rows, in expert order
// (kernels/exl3r4d/launch.c:14-15 clamps the runs); then, for each GEMM, the chunks dealt to the 8 XCDs in contiguous
// ranges of about equal cost (a chunk of t tiles: W + t; its midpoint in cost order picks the XCD); then each row's
// owner. Its own kernel (k_plan), or the first workgroup of k_rot's launch, running beside the rotation.
constexpr int PF_TILES = EXL3C4_PF_ROWS / 16;                     // row tiles a chunk holds at most
// The rows a chunk of this launch holds: seven row tiles where both GEMMs decode at K <= 4 (their loops then hold
// seven tiles of accumulators in the 128 registers of 4 waves a SIMD), six at larger K (seven would spill there)
__device__ __forceinline__ int pf_rows(const Exl3c4Launch& a) {
    return a.bits <= 4 && a.dn_bits <= 4 ? EXL3C4_PF_ROWS : EXL3C4_PF_ROWS_WIDE;
}
// The plan's chunk order of one GEMM (gate_up 0, down 1): max_chunks entries after the chunk entries.
__device__ __forceinline__ const int32_t* pf_order(const Exl3c4Launch& a, int gemm) {
    return a.plan + EXL3C4_PF_PLAN_HDR + 4 * a.max_chunks + gemm * a.max_chunks;
}
// The XCD of a chunk whose cost starts at p_excl, of a GEMM whose chunks cost total: its cost midpoint's eighth,
// min(7, floor(8 (2 p_excl + cost) / (2 total))), counted as the j = 1..7 with 2 j total <= 8 (2 p_excl + cost)
// (comparisons, no division).
__device__ __forceinline__ int pf_xcd_of(int p_excl, int cost, int total) {
    const int64_t m8 = 8ll * (2ll * p_excl + cost), t2 = 2ll * max(total, 1);
    int x = 0;
#pragma unroll
    for (int j = 1; j < 8; ++j) x += m8 >= j * t2 ? 1 : 0;
    return x;
}
// The plan for any number of experts: a block of NT experts at a time, the chunk entries written, then read back for
// the XCD deal, the orders and the rows' owners (a round trip of global memory for each).
template <int NT> __device__ __forceinline__ void plan_generic(const Exl3c4Launch& a) {
    __shared__ int scan[NT];
    __shared__ int carry_s, tiles_s, cut_s, cnt_g[8], cnt_d[8];
    __shared__ int cur_g[8][PF_TILES], cur_d[8][PF_TILES];           // per (XCD, tiles): chunk counts, then cursors
    const int tid = threadIdx.x;
    const int R = pf_rows(a);                                      // a chunk's rows at most
    if (tid == 0) {
        carry_s = tiles_s = 0;
        cut_s = 0x7FFFFFFF;
    }
    if (tid < 8) cnt_g[tid] = cnt_d[tid] = 0;
    if (tid < 8 * PF_TILES) cur_g[tid / PF_TILES][tid % PF_TILES] = cur_d[tid / PF_TILES][tid % PF_TILES] = 0;
    __syncthreads();
    int4* ent = (int4*)(a.plan + EXL3C4_PF_PLAN_HDR);
    for (int base = 0; base < a.n_expert; base += NT) {
        const int e = base + tid;
        int lo = 0, hi = 0, n = 0;
        if (e < a.n_expert) {
            lo = min(max(a.off[e], 0), a.T);
            hi = min(max(a.off[e + 1], lo), a.T);
            n = (hi - lo + R - 1) / R;
        }
        scan[tid] = n;
        __syncthreads();
        for (int d = 1; d < NT; d <<= 1) {                     // inclusive scan
            const int t = tid >= d ? scan[tid - d] : 0;
            __syncthreads();
            scan[tid] += t;
            __syncthreads();
        }
        const int first = carry_s + scan[tid] - n;
        int tiles = 0;
        for (int q = 0; q < n; ++q) {
            const int at = first + q;
            if (at < a.max_chunks) {
                const int r0 = lo + q * R, rows = min(R, hi - r0);
                ent[at] = make_int4(e, r0, rows, 0);
                tiles += (rows + 15) >> 4;
            }
        }
        if (tiles) atomicAdd(&tiles_s, tiles);
        __syncthreads();
        if (tid == NT - 1) carry_s += scan[NT - 1];
        __syncthreads();
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");             // the entries, read by other threads below
    __syncthreads();
    int nch = min(carry_s, a.max_chunks);
    // the tile budget, T / 16 + min(n_expert, T) (the launch's grid holds the chunks of at most that many tiles, with
    // max_chunks; runs that do not overlap never pass it): the chunks from the first whose running tiles pass it are
    // dropped, as those past max_chunks are
    const int budget = a.T / 16 + min(a.n_expert, a.T);
    if (tiles_s > budget) {                                       // uniform
        int run = 0;
        for (int base = 0; base < nch; base += NT) {
            const int c = base + tid;
            const int t = c < nch ? (ent[c].z + 15) >> 4 : 0;
            scan[tid] = t;
            __syncthreads();
            for (int d = 1; d < NT; d <<= 1) {
                const int u = tid >= d ? scan[tid - d] : 0;
                __syncthreads();
                scan[tid] += u;
                __syncthreads();
            }
            if (c < nch && run + scan[tid] > budget) atomicMin(&cut_s, c);
            run += scan[NT - 1];
            __syncthreads();
        }
        if (tid == 0) tiles_s = 0;
        __syncthreads();
        nch = min(nch, cut_s);
        int t = 0;                                                // the kept chunks' tiles
        for (int c = tid; c < nch; c += NT) t += (ent[c].z + 15) >> 4;
        if (t) atomicAdd(&tiles_s, t);
        __syncthreads();
    }
    const int tot_g = EXL3C4_PF_W_GU * nch + tiles_s, tot_d = EXL3C4_PF_W_DN * nch + tiles_s;
    // the chunks' tile prefix
    int carry = 0;
    for (int base = 0; base < nch; base += NT) {
        const int c = base + tid;
        const int t = c < nch ? (ent[c].z + 15) >> 4 : 0;
        scan[tid] = t;
        __syncthreads();
        for (int d = 1; d < NT; d <<= 1) {
            const int u = tid >= d ? scan[tid - d] : 0;
            __syncthreads();
            scan[tid] += u;
            __syncthreads();
        }
        if (c < nch) {
            const int p = carry + scan[tid] - t;                  // tiles of the chunks before c
            const int xg = pf_xcd_of(EXL3C4_PF_W_GU * c + p, EXL3C4_PF_W_GU + t, tot_g);
            const int xd = pf_xcd_of(EXL3C4_PF_W_DN * c + p, EXL3C4_PF_W_DN + t, tot_d);
            atomicAdd(&cnt_g[xg], 1);
            atomicAdd(&cnt_d[xd], 1);
            atomicAdd(&cur_g[xg][t - 1], 1);
            atomicAdd(&cur_d[xd][t - 1], 1);
            ent[c].w = xg | (xd << 8);
        }
        carry += scan[NT - 1];
        __syncthreads();
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");             // the entries' XCDs, read by other threads below
    __syncthreads();
    if (tid < 16) __hip_atomic_store(a.plan + EXL3C4_PF_CUR + 32 * tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
        a.plan[0] = nch;
        a.plan[EXL3C4_PF_SPAN] = 0;                               // the rows' owners in row_info
        int bg = 0, bd = 0;
        for (int x = 0; x < 8; ++x) {
            a.plan[EXL3C4_PF_XCD_GU + x] = bg;
            a.plan[EXL3C4_PF_XCD_DN + x] = bd;
            bg += cnt_g[x];
            bd += cnt_d[x];
        }
        a.plan[EXL3C4_PF_XCD_GU + 8] = bg;
        a.plan[EXL3C4_PF_XCD_DN + 8] = bd;
    }
    // each GEMM's order: inside an XCD's range, chunks of more row tiles first (the longest units start first, so
    // the range ends on short ones); chunks of equal tiles in any order (where a unit runs changes no bits)
    if (tid < 16) {
        int (*cur)[PF_TILES] = tid < 8 ? cur_g : cur_d;
        const int x = tid & 7;
        int at = 0;
        for (int y = 0; y < x; ++y) at += (tid < 8 ? cnt_g : cnt_d)[y];
        for (int k = PF_TILES - 1; k >= 0; --k) {
            const int n = cur[x][k];
            cur[x][k] = at;
            at += n;
        }
    }
    __syncthreads();
    int32_t* ord_g = (int32_t*)(ent + a.max_chunks);
    int32_t* ord_d = ord_g + a.max_chunks;
    for (int c = tid; c < nch; c += NT) {
        const int w = ent[c].w, t = (ent[c].z + 15) >> 4;
        ord_g[atomicAdd(&cur_g[w & 255][t - 1], 1)] = c;
        ord_d[atomicAdd(&cur_d[w >> 8][t - 1], 1)] = c;
    }
    // each row's owner (row_info[i] = {e or -1, 0}): every row -1 first, then a chunk's rows its expert; the first
    // stores complete before any thread passes the barrier, so a row's last store is its owner's
    for (int i = tid; i < a.T; i += NT) *(int2*)(a.row_info + 2 * i) = make_int2(-1, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int c = tid; c < nch; c += NT) {
        const int4 en = ent[c];
        for (int r = 0; r < en.z; ++r) a.row_info[2 * (en.y + r)] = en.x;
    }
}
// An inclusive prefix sum over a workgroup of NT threads (NT / 64 waves) of (tiles << 32 | chunks) pairs: within each
// wave by lane shuffles, then the waves' totals through LDS (wsum: NT / 64 entries); total: the workgroup's sum. Two
// barriers.
template <int NT> __device__ __forceinline__ int64_t block_scan64(int64_t v, int64_t* wsum, int64_t& total) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int64_t t = __shfl_up(v, d);
        if (lane >= d) v += t;
    }
    if (lane == 63) wsum[w] = v;
    __syncthreads();
    int64_t pre = 0;
    total = 0;
#pragma unroll
    for (int j = 0; j < NT / 64; ++j) {
        pre += j < w ? wsum[j] : 0;
        total += wsum[j];
    }
    __syncthreads();                                              // wsum is read before the next scan writes it
    return v + pre;
}
// The plan for up to EPT x NT experts, thread tid taking experts tid, NT + tid, ... through every phase (their runs,
// first chunks and tile prefixes kept in LDS, each entry written and read by its own thread): one round of loads (the
// offsets), then scans, LDS counters and stores only -- nothing the workgroup writes to global memory is read back, so
// no phase waits for its stores. The same plan as plan_generic: chunks in expert order, each expert's run clamped to
// [0, T) and cut into chunks of at most pf_rows rows (all full but the last), the chunks past max_chunks
// dropped (their rows' owner -1); each chunk's XCDs from its cost midpoint; each GEMM's order by tiles inside an
// XCD's range; the rows' owners.
// The plan for up to EPT x NT experts, thread tid taking experts tid, NT + tid, ... (their clamped runs, first chunks
// and tile prefixes kept in LDS, each entry written and read by its own thread): one round of loads (the offsets),
// then scans, LDS counters and stores only -- nothing the workgroup writes to global memory is read back, so no phase
// waits for its stores. The same plan as plan_generic: chunks in expert order, each expert's run clamped to [0, T) and
// cut into chunks of at most pf_rows rows (all full but the last), the chunks past max_chunks dropped; each
// chunk's XCDs from its cost midpoint; each GEMM's order by tiles inside an XCD's range. A thread's chunks of one
// expert fall into runs of equal (XCD, tiles) -- the XCD grows with the chunk index -- and each run costs one LDS
// atomic: the counts added when a run ends, a run's slots in the order taken by one atomicAdd of its length. The rows'
// owners: when the offsets ascend and no chunk is dropped, the held rows are the one span [off[0], off[n_expert])
// (clamped), recorded in the plan's header (EXL3C4_PF_SPAN) for zero_dead_rows; otherwise each row's owner in
// row_info, as plan_generic writes it.
template <int NT, int EPT> __device__ __forceinline__ void plan_fast(const Exl3c4Launch& a) {
    __shared__ int64_t wsum[NT / 64];
    __shared__ int cnt_g[8], cnt_d[8], tk_s, desc_s, cut_s;
    __shared__ int cur_g[8][PF_TILES], cur_d[8][PF_TILES];           // per (XCD, tiles): chunk counts, then cursors
    __shared__ int s_lo[EPT * NT], s_hi[EPT * NT], s_first[EPT * NT], s_tf[EPT * NT];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int R = pf_rows(a), RT = R >> 4;                         // a chunk's rows and tiles at most
    if (tid < 8) cnt_g[tid] = cnt_d[tid] = 0;
    if (tid == 0) {
        tk_s = desc_s = 0;
        cut_s = 0x7FFFFFFF;
    }
    if (tid < 8 * PF_TILES) cur_g[tid / PF_TILES][tid % PF_TILES] = cur_d[tid / PF_TILES][tid % PF_TILES] = 0;
    int lo[EPT], hi[EPT];
#pragma unroll
    for (int k = 0; k < EPT; ++k) {                               // the offsets: one round of loads
        const int e = k * NT + tid;
        lo[k] = e < a.n_expert ? a.off[e] : 0;
        hi[k] = e < a.n_expert ? a.off[e + 1] : 0;
    }
    int64_t carry = 0;
    bool desc = false;                                            // an offset below the one before it
#pragma unroll
    for (int k = 0; k < EPT; ++k) {
        if (k * NT >= a.n_expert) break;                          // uniform
        const int e = k * NT + tid;
        desc = desc || (e < a.n_expert && hi[k] < lo[k]);
        const int l = min(max(lo[k], 0), a.T), h = min(max(hi[k], l), a.T);
        const int n = e < a.n_expert ? (h - l + R - 1) / R : 0;
        const int rem = h - l - (n - 1) * R;                      // the last chunk's rows
        const int tiles = n ? (n - 1) * RT + ((rem + 15) >> 4) : 0;
        const int64_t v = ((int64_t)tiles << 32) | (uint32_t)n;
        int64_t blk;
        const int64_t ex = carry + block_scan64<NT>(v, wsum, blk) - v;
        s_lo[e] = l;
        s_hi[e] = h;
        s_first[e] = (int)(ex & 0xFFFFFFFF);
        s_tf[e] = (int)(ex >> 32);                                // tiles of the chunks before this expert's
        carry += blk;
    }
    if (desc) desc_s = 1;
    // the tile budget, T / 16 + min(n_expert, T) (the launch's grid holds the chunks of at most that many tiles, with
    // max_chunks; runs that do not overlap never pass it): the chunks from the first whose running tiles pass it are
    // dropped, as those past max_chunks are -- found by the one expert whose chunks cross it
    const int budget = a.T / 16 + min(a.n_expert, a.T);
    if ((int)(carry >> 32) > budget) {                            // uniform
#pragma unroll 1
        for (int k = 0; k < EPT; ++k) {
            const int e = k * NT + tid;
            if (e >= a.n_expert) break;
            const int l = s_lo[e], h = s_hi[e], f = s_first[e], tf = s_tf[e];
            for (int r0 = l, at = f, p = tf; r0 < h; r0 += R, ++at, p += RT)
                if (p + ((min(R, h - r0) + 15) >> 4) > budget) {
                    atomicMin(&cut_s, at);
                    break;
                }
        }
        __syncthreads();
    }
    const int nch_all = (int)(carry & 0xFFFFFFFF), nch = min(min(nch_all, a.max_chunks), cut_s);
    // the kept chunks' tiles: all of them unless chunks were dropped (those come last in chunk order)
    int tiles_kept = (int)(carry >> 32);
    if (nch < nch_all) {                                          // uniform
        int t = 0;
#pragma unroll 1
        for (int k = 0; k < EPT; ++k) {
            const int e = k * NT + tid, l = s_lo[e], h = s_hi[e], f = s_first[e];
            for (int r0 = l, at = f; r0 < h && at < nch; r0 += R, ++at)
                t += (min(R, h - r0) + 15) >> 4;
        }
        if (t) atomicAdd(&tk_s, t);
        __syncthreads();
        tiles_kept = tk_s;
    }
    const int tot_g = EXL3C4_PF_W_GU * nch + tiles_kept, tot_d = EXL3C4_PF_W_DN * nch + tiles_kept;
    // each chunk's entry {e, first row, rows, XCD of gate_up | XCD of down << 8}; the (XCD, tiles) counts a run at a
    // time (run: consecutive chunks of the thread's expert of one class, kg / kd = XCD x PF_TILES + tiles - 1)
    int4* ent = (int4*)(a.plan + EXL3C4_PF_PLAN_HDR);
#pragma unroll 1
    for (int k = 0; k < EPT; ++k) {
        if (k * NT >= a.n_expert) break;                          // uniform
        const int e = k * NT + tid, l = s_lo[e], h = s_hi[e], f = s_first[e], tf = s_tf[e];
        int kg = -1, kd = -1, ng = 0, nd = 0;
        for (int r0 = l, at = f, p = tf; r0 < h && at < nch; r0 += R, ++at, p += RT) {
            const int rows = min(R, h - r0), t = (rows + 15) >> 4;   // earlier chunks: full
            const int xg = pf_xcd_of(EXL3C4_PF_W_GU * at + p, EXL3C4_PF_W_GU + t, tot_g);
            const int xd = pf_xcd_of(EXL3C4_PF_W_DN * at + p, EXL3C4_PF_W_DN + t, tot_d);
            ent[at] = make_int4(e, r0, rows, xg | (xd << 8));
            const int cg = xg * PF_TILES + t - 1, cd = xd * PF_TILES + t - 1;
            if (cg != kg) {
                if (ng) {
                    atomicAdd(&cur_g[0][0] + kg, ng);
                    atomicAdd(&cnt_g[kg / PF_TILES], ng);
                }
                kg = cg;
                ng = 0;
            }
            if (cd != kd) {
                if (nd) {
                    atomicAdd(&cur_d[0][0] + kd, nd);
                    atomicAdd(&cnt_d[kd / PF_TILES], nd);
                }
                kd = cd;
                nd = 0;
            }
            ++ng;
            ++nd;
        }
        if (ng) {
            atomicAdd(&cur_g[0][0] + kg, ng);
            atomicAdd(&cnt_g[kg / PF_TILES], ng);
        }
        if (nd) {
            atomicAdd(&cur_d[0][0] + kd, nd);
            atomicAdd(&cnt_d[kd / PF_TILES], nd);
        }
    }
    __syncthreads();
    const bool span = desc_s == 0 && nch == nch_all;              // the held rows: one span
    if (tid < 16) __hip_atomic_store(a.plan + EXL3C4_PF_CUR + 32 * tid, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (tid == 0) {
        a.plan[0] = nch;
        a.plan[EXL3C4_PF_SPAN] = span ? 1 : 0;
        a.plan[EXL3C4_PF_SPAN + 1] = min(max(a.off[0], 0), a.T);
        a.plan[EXL3C4_PF_SPAN + 2] = min(max(a.off[a.n_expert], 0), a.T);
        int bg = 0, bd = 0;
        for (int x = 0; x < 8; ++x) {
            a.plan[EXL3C4_PF_XCD_GU + x] = bg;
            a.plan[EXL3C4_PF_XCD_DN + x] = bd;
            bg += cnt_g[x];
            bd += cnt_d[x];
        }
        a.plan[EXL3C4_PF_XCD_GU + 8] = bg;
        a.plan[EXL3C4_PF_XCD_DN + 8] = bd;
    }
    // each GEMM's order: inside an XCD's range, chunks of more row tiles first (the longest units start first, so
    // the range ends on short ones); chunks of equal tiles in any order (where a unit runs changes no bits)
    if (tid < 16) {
        int (*cur)[PF_TILES] = tid < 8 ? cur_g : cur_d;
        const int x = tid & 7;
        int at = 0;
        for (int y = 0; y < x; ++y) at += (tid < 8 ? cnt_g : cnt_d)[y];
        for (int k = PF_TILES - 1; k >= 0; --k) {
            const int c = cur[x][k];
            cur[x][k] = at;
            at += c;
        }
    }
    __syncthreads();
    int32_t* ord_g = (int32_t*)(ent + a.max_chunks);
    int32_t* ord_d = ord_g + a.max_chunks;
    // a run's slots: one atomicAdd of its length when it ends, then its chunks (consecutive indices) in them
    auto place = [&](int32_t* ord, int* cur, int key, int n, int at_end) {
        const int base = atomicAdd(cur + key, n);
        for (int j = 0; j < n; ++j) ord[base + j] = at_end - n + j;
    };
#pragma unroll 1
    for (int k = 0; k < EPT; ++k) {
        if (k * NT >= a.n_expert) break;                          // uniform
        const int e = k * NT + tid, l = s_lo[e], h = s_hi[e], f = s_first[e], tf = s_tf[e];
        int kg = -1, kd = -1, ng = 0, nd = 0, at = f;
        for (int r0 = l, p = tf; r0 < h && at < nch; r0 += R, ++at, p += RT) {
            const int t = (min(R, h - r0) + 15) >> 4;
            const int cg = pf_xcd_of(EXL3C4_PF_W_GU * at + p, EXL3C4_PF_W_GU + t, tot_g) * PF_TILES + t - 1;
            const int cd = pf_xcd_of(EXL3C4_PF_W_DN * at + p, EXL3C4_PF_W_DN + t, tot_d) * PF_TILES + t - 1;
            if (cg != kg) {
                if (ng) place(ord_g, &cur_g[0][0], kg, ng, at);
                kg = cg;
                ng = 0;
            }
            if (cd != kd) {
                if (nd) place(ord_d, &cur_d[0][0], kd, nd, at);
                kd = cd;
                nd = 0;
            }
            ++ng;
            ++nd;
        }
        if (ng) place(ord_g, &cur_g[0][0], kg, ng, at);
        if (nd) place(ord_d, &cur_d[0][0], kd, nd, at);
    }
    if (span) return;                                             // uniform
    // each row's owner (row_info[i] = {e or -1, 0}): every row -1, then, once those stores have completed, the rows
    // of the kept chunks' runs their expert, written by the wave's lanes side by side one expert at a time (a row two
    // runs hold, from offsets that do not ascend, takes either expert)
    for (int i = tid; i < a.T; i += NT) *(int2*)(a.row_info + 2 * i) = make_int2(-1, 0);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
#pragma unroll 1
    for (int k = 0; k < EPT; ++k) {
        const int e0 = k * NT + 64 * wave;
        if (e0 >= a.n_expert) break;                              // uniform
        const int ml = s_lo[e0 + lane];                           // the wave's 64 experts, lane-parallel
        const int mh = min(s_hi[e0 + lane], ml + max(0, nch - s_first[e0 + lane]) * R);   // past it:
        for (int j = 0; j < 64; ++j) {                                                                // dropped
            const int l = __builtin_amdgcn_readlane(ml, j), hk = __builtin_amdgcn_readlane(mh, j);   // chunks' rows,
            for (int r = l + lane; r < hk; r += 64) a.row_info[2 * r] = e0 + j;                      // left -1
        }
    }
}
template <int NT> __device__ __forceinline__ void plan_body(const Exl3c4Launch& a) {
    if (a.n_expert <= 4 * NT) plan_fast<NT, 4>(a);
    else plan_generic<NT>(a);
}
__global__ __launch_bounds__(1024) void k_plan(const Exl3c4Launch a) { plan_body<1024>(a); }



// had128 over 128-blocks held 8 consecutive elements a lane: lane l of a 16-lane row holds the elements 8 g .. 8 g + 7
// of its block, g = rot_group(l) = l ^ 3 where bit 2 of l is set, else l. The stages h = 1, 2, 4 run inside the lane;
// h = 8, 16, 32, 64 (bits 0 .. 3 of g) pair lane l with l ^ 1, l ^ 2, l ^ 7, l ^ 8 -- the lanes whose g differs in that
// bit alone, each one DPP move (quad_perm, quad_perm, row_half_mirror, row_ror 8) -- as in had128_wave: v_fmac by
// c = -1 on the lanes whose g has the stage's bit set leaves them the NEGATED result, the partner (same lower bits of
// g) carries the same sign, and the final multiply by -1/sqrt(128) where popcount(g) is odd undoes it, as an fma with
// +0 (an exact zero leaves as +0, as had128_wave's does). The reference's stages in its order with its roundings
// (common/exl3_decode.c:172-189), so the same values, and the same bits but for the sign of zeros that had128_wave
// states.
__device__ __forceinline__ int rot_group(int l) { return l ^ (((l >> 2) & 1) * 3); }
#define HAD_DPP8_OP(I, CTRL) "v_fmac_f32_dpp %" #I ", %" #I ", %8 " CTRL " row_mask:0xf bank_mask:0xf\n\t"
// one stage over the 8 values: a lane's v[j] was written 8 moves before it is read, so one s_nop (the DPP read-after-
// VALU-write distance) opens the block and none sits between its moves
#define HAD_DPP8(v, c, CTRL)                                                                                   \
    asm volatile("s_nop 1\n\t" HAD_DPP8_OP(0, CTRL) HAD_DPP8_OP(1, CTRL) HAD_DPP8_OP(2, CTRL)               \
                 HAD_DPP8_OP(3, CTRL) HAD_DPP8_OP(4, CTRL) HAD_DPP8_OP(5, CTRL) HAD_DPP8_OP(6, CTRL)           \
                 HAD_DPP8_OP(7, CTRL)                                                                         \
                 : "+v"(v[0]), "+v"(v[1]), "+v"(v[2]), "+v"(v[3]), "+v"(v[4]), "+v"(v[5]), "+v"(v[6]),       \
                   "+v"(v[7])                                                                                 \
                 : "v"(c))
struct RotSigns { float c1, c2, c4, c8, sc; };
__device__ __forceinline__ RotSigns rot_signs(int g) {
    return RotSigns{ (g & 1) ? -1.f : 1.f, (g & 2) ? -1.f : 1.f, (g & 4) ? -1.f : 1.f, (g & 8) ? -1.f : 1.f,
                     (__builtin_popcount(g) & 1) ? -kHadScale : kHadScale };
}
template <int H0 = 1>                                             // the first in-lane stage not yet done
__device__ __forceinline__ void had128_x8(float (&v)[8], const RotSigns& k) {
#pragma unroll
    for (int h = H0; h < 8; h <<= 1)
#pragma unroll
        for (int j = 0; j < 8; ++j)
            if (!(j & h)) {
                const float a = v[j], b = v[j + h];
                v[j] = a + b;
                v[j + h] = a - b;
            }
    HAD_DPP8(v, k.c1, "quad_perm:[1,0,3,2]");
    HAD_DPP8(v, k.c2, "quad_perm:[2,3,0,1]");
    HAD_DPP8(v, k.c4, "row_half_mirror");
    HAD_DPP8(v, k.c8, "row_ror:8");
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = __builtin_fmaf(v[j], k.sc, 0.f);   // + 0: an exact zero leaves as +0
}

// 8 consecutive halves at p as 4 dwords (16-byte aligned: one load; else eight)
__device__ __forceinline__ void load8w(const uint16_t* p, bool wide, uint32_t (&w)[4]) {
    if (wide) {
        const uint4 q = *(const uint4*)p;
        w[0] = q.x; w[1] = q.y; w[2] = q.z; w[3] = q.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) w[j] = (uint32_t)ldg16(p, 2 * j) | ((uint32_t)ldg16(p, 2 * j + 1) << 16);
    }
}

// The rotation into scratch, ROT_ROWS consecutive sorted rows a wave, 8 consecutive elements a lane: a pass covers 4
// 128-blocks of each half of each row (one 16-byte load of x, one of each scale and one store a half a lane), and the
// loads of up to ROT_PASSES passes of all the wave's rows go out together: gate_up's xr (halves 0 and 1 from the same
// token row: suh, suh1 of the row's expert) or down's rotated h (one half: down's suh, sorted rows in). A wave can run
// several rows' chains (owner, class tables, loads, stores) side by side; one row a wave measured fastest (2048
// tokens: 45.2 us against 46.9 for two rows and 54.2 for four: more rows a wave cost resident waves). The stores are
// non-temporal (xr is read once, by the GEMM, after the 4 MiB L2s have turned over). The first step f16(x su) is one f16 multiply (v_pk_mul_f16: the exact
// product rounded once, as f16(f32(x) f32(su)) rounds it; bf16 x: in f32, then rounded). The rows are dealt to the
// XCDs in contiguous ranges, so a run's rows (one expert's scales) share an L2. Rows no run holds are not written
// (nothing reads them); a negative sorted_tok gives zeros.
constexpr int ROT_PASSES = 2, ROT_ROWS = 1;
// f32 (lo of w) + f32 (hi of w) and f32 (lo) - f32 (hi) of a dword of two f16 values: each one v_fma_mix_f32 (the f16
// sources taken exactly, one rounding), the first butterfly stage of two neighbours straight from their packed f16
// product -- as the f16 -> f32 conversions then an f32 add and subtract would round them.
__device__ __forceinline__ void mix_sum_diff(uint32_t w, float& sum, float& dif) {
    asm("v_fma_mix_f32 %0, %2, 1.0, %2 op_sel:[0,0,1] op_sel_hi:[1,0,1]\n\t"
        "v_fma_mix_f32 %1, %2, 1.0, -%2 op_sel:[0,0,1] op_sel_hi:[1,0,1]"
        : "=&v"(sum), "=v"(dif) : "v"(w));
}

// One wave's R rows of one class (C columns): per pass each lane's 8 consecutive columns of each half of each row
// (BF: x in bf16), as described at k_rot. Row r: x[r] its input row, s0[r] / s1[r] its expert's scales, out[r] its xr
// row; zero[r]: written as zeros (a negative sorted_tok; its loads read a valid row, unused); wr[r]: written at all.
template <bool BF, int HALVES, int R>
__device__ __forceinline__ void rot_passes(const uint16_t* const (&x)[R], const uint16_t* const (&s0)[R],
                                           const uint16_t* const (&s1)[R], uint16_t* const (&out)[R],
                                           const bool (&zero)[R], const bool (&wr)[R], int C, int npass, int lcol,
                                           int g, bool xw, bool sw, const RotSigns& ks) {
    for (int p0 = 0; p0 < npass; p0 += ROT_PASSES) {
        uint32_t xq[R][ROT_PASSES][4], sq[R][2][ROT_PASSES][4];
#pragma unroll
        for (int r = 0; r < R; ++r)
#pragma unroll
            for (int q = 0; q < ROT_PASSES; ++q) {
                int col = (p0 + q) * 512 + lcol;
                col = col < C ? col : 8 * g;                        // past the row: reload the first block (unused)
                load8w(x[r] + col, xw, xq[r][q]);
                load8w(s0[r] + col, sw, sq[r][0][q]);
                if (HALVES == 2) load8w(s1[r] + col, sw, sq[r][1][q]);
            }
#pragma unroll
        for (int r = 0; r < R; ++r) {
            if (!wr[r]) continue;                                 // uniform
#pragma unroll
            for (int m = 0; m < HALVES; ++m) {
#pragma unroll
                for (int q = 0; q < ROT_PASSES; ++q) {
                    if (p0 + q >= npass) break;
                    float v[8];
                    if (BF) {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const uint32_t xb = xq[r][q][j], sb = sq[r][m][q][j];
                            v[2 * j] = h2f(f2h(bf2f((uint16_t)xb) * h2f((uint16_t)sb)));
                            v[2 * j + 1] = h2f(f2h(bf2f((uint16_t)(xb >> 16)) * h2f((uint16_t)(sb >> 16))));
                        }
                        had128_x8(v, ks);
                    } else {
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const half2_t pr = __builtin_bit_cast(half2_t, xq[r][q][j]) *
                                               __builtin_bit_cast(half2_t, sq[r][m][q][j]);
                            mix_sum_diff(__builtin_bit_cast(uint32_t, pr), v[2 * j], v[2 * j + 1]);   // stage h = 1
                        }
                        had128_x8<2>(v, ks);
                    }
                    u32x4_t o;                                    // (a v_cvt_pk_f16_f32 of the scaled values:
#pragma unroll                                                    // the bits are checked against prep_gu's)
                    for (int j = 0; j < 4; ++j) {
                        typedef float float2v __attribute__((ext_vector_type(2)));
                        const half2_t hv = __builtin_convertvector(float2v{ v[2 * j], v[2 * j + 1] }, half2_t);
                        o[j] = zero[r] ? 0u : __builtin_bit_cast(uint32_t, hv);
                    }
                    const int col = (p0 + q) * 512 + lcol;
                    if (col < C) __builtin_nontemporal_store(o, (u32x4_t*)(out[r] + m * C + col));
                }
            }
        }
    }
}

// The owners of the R sorted rows i0 .. i0 + R - 1 (-1: no run holds the row, or it lies past T): owner_wave's
// search, its one round of loads shared by the rows (off[] read once, a ballot count a row).
template <int R>
__device__ __forceinline__ void owner_rows(const int32_t* off, int n_expert, int i0, int T, int lane, int (&e)[R]) {
    constexpr int OJ = 9;
    if (n_expert < 64 * OJ) {
        int o[OJ];
#pragma unroll
        for (int j = 0; j < OJ; ++j) o[j] = off[min(lane + 64 * j, n_expert)];
#pragma unroll
        for (int r = 0; r < R; ++r) {
            const int i = i0 + r;
            int cnt = 0;
#pragma unroll
            for (int j = 0; j < OJ; ++j) {
                const int ej = lane + 64 * j;
                cnt += __popcll(__ballot(ej >= 1 && ej <= n_expert && o[j] <= i));
            }
            const int er = min(cnt, n_expert - 1);
            int lo = 0, hi = 0;
#pragma unroll
            for (int j = 0; j < OJ; ++j) {
                if ((er >> 6) == j) lo = __builtin_amdgcn_readlane(o[j], er & 63);
                if (((er + 1) >> 6) == j) hi = __builtin_amdgcn_readlane(o[j], (er + 1) & 63);
            }
            e[r] = (i < T && lo <= i && i < hi) ? er : -1;
        }
        return;
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
        e[r] = i0 + r < T ? __builtin_amdgcn_readfirstlane(owner_wave(off, n_expert, i0 + r, lane)) : -1;
}

template <bool BF, int HALVES>
__device__ __forceinline__ void rot_rows(const Exl3c4Launch& a, int i0, const int (&e)[ROT_ROWS],
                                         const int (&tok)[ROT_ROWS], int lane) {
    // the rows' class: one class for all held rows (the usual case) runs them side by side, else one at a time
    int eb = -1;
#pragma unroll
    for (int r = ROT_ROWS - 1; r >= 0; --r) eb = e[r] >= 0 ? e[r] : eb;
    if (eb < 0) return;                                           // no row held
    bool same = true;
#pragma unroll
    for (int r = 0; r < ROT_ROWS; ++r) same = same && (e[r] < 0 || class_of(a, e[r]) == class_of(a, eb));
    const int g = rot_group(lane & 15), lcol = 128 * (lane >> 4) + 8 * g;   // the lane's columns in a pass
    const RotSigns ks = rot_signs(g);
    const bool xw = (((uintptr_t)a.x | (uintptr_t)(a.x_pitch * 2)) & 15) == 0;
    auto row = [&](int r, const Exl3c4DevClass& K, const uint16_t*& x, const uint16_t*& s0, const uint16_t*& s1,
                   uint16_t*& out, bool& zero, bool& wr) {
        const int er = e[r] >= 0 ? e[r] : eb, i = i0 + r;
        const int64_t jx = entry_of(a, er);
        int64_t src = HALVES == 2 ? (tok[r] < 0 ? 0 : tok[r] / a.top_k) : min(i, a.T - 1);
        src = src < a.x_rows ? src : a.x_rows - 1;
        x = (const uint16_t*)a.x + src * a.x_pitch;
        s0 = (const uint16_t*)tab_entry(K.suh, K.suh_s, jx);
        s1 = HALVES == 2 ? (const uint16_t*)tab_entry(K.suh1, K.suh1_s, jx) : s0;
        out = (uint16_t*)a.y + (int64_t)min(i, a.T - 1) * a.y_pitch;
        zero = tok[r] < 0;
        wr = e[r] >= 0;
    };
    if (same) {
        const Exl3c4DevClass& K = a.cls[class_of(a, eb)];
        const uint16_t* x[ROT_ROWS];
        const uint16_t* s0[ROT_ROWS];
        const uint16_t* s1[ROT_ROWS];
        uint16_t* out[ROT_ROWS];
        bool zero[ROT_ROWS], wr[ROT_ROWS];
        bool sw = true;
#pragma unroll
        for (int r = 0; r < ROT_ROWS; ++r) {
            row(r, K, x[r], s0[r], s1[r], out[r], zero[r], wr[r]);
            sw = sw && ((((uintptr_t)s0[r] | (uintptr_t)s1[r]) & 15) == 0);
        }
        const int C = K.cols, npass = (C / 128 + 3) / 4;
        rot_passes<BF, HALVES, ROT_ROWS>(x, s0, s1, out, zero, wr, C, npass, lcol, g, xw, sw, ks);
        return;
    }
#pragma unroll 1
    for (int r = 0; r < ROT_ROWS; ++r) {
        if (e[r] < 0) continue;
        const Exl3c4DevClass& K = a.cls[class_of(a, e[r])];
        const uint16_t* x[1];
        const uint16_t* s0[1];
        const uint16_t* s1[1];
        uint16_t* out[1];
        bool zero[1], wr[1];
        row(r, K, x[0], s0[0], s1[0], out[0], zero[0], wr[0]);
        const bool sw = (((uintptr_t)s0[0] | (uintptr_t)s1[0]) & 15) == 0;
        const int C = K.cols, npass = (C / 128 + 3) / 4;
        rot_passes<BF, HALVES, 1>(x, s0, s1, out, zero, wr, C, npass, lcol, g, xw, sw, ks);
    }
}

__global__ __launch_bounds__(256) void k_rot(const Exl3c4Launch a) {
    if (a.plan && blockIdx.x == 0) {                              // the launch's first workgroup plans the GEMMs
        plan_body<256>(a);
        return;
    }
    const int lane = threadIdx.x & 63;
    const int gb = (int)blockIdx.x - (a.plan ? 1 : 0);
    const int nwg = (a.T + 4 * ROT_ROWS - 1) / (4 * ROT_ROWS), per_xcd = (nwg + 7) / 8;
    const int wg = (gb & 7) * per_xcd + (gb >> 3);
    // the rows, their owners and their sorted_tok taken wave-uniform: the class descriptor and the rows' entries are
    // then scalar loads that go out together, not vector loads each waited for
    const int i0 = __builtin_amdgcn_readfirstlane((wg * 4 + (int)(threadIdx.x >> 6)) * ROT_ROWS);
    if (wg >= nwg || i0 >= a.T) return;
    const int tok_v = a.sorted[min(i0 + (lane & (ROT_ROWS - 1)), a.T - 1)];   // lane r: row i0 + r's, out with the
    int e[ROT_ROWS], tok[ROT_ROWS];                                             // owner search's loads
    owner_rows<ROT_ROWS>(a.off, a.n_expert, i0, a.T, lane, e);   // -1: a row no run holds, not written
#pragma unroll
    for (int r = 0; r < ROT_ROWS; ++r) tok[r] = __builtin_amdgcn_readlane(tok_v, r);
    if (a.h_from_gu == 2) {                                       // here: 2 halves for gate_up's xr, 1 for down's h
        if (a.x_dtype == EXL3C4_BF16) rot_rows<true, 2>(a, i0, e, tok, lane);
        else rot_rows<false, 2>(a, i0, e, tok, lane);
    } else {
        rot_rows<false, 1>(a, i0, e, tok, lane);
    }
}

// Zero the 128-blocks of y of the rows no run holds (the prefill GEMMs write only their chunks' rows): the
// PF_TAIL_WG workgroups from a.tail_from of the last GEMM's launch, wave w of workgroup z taking rows z * NW + w,
// then every PF_TAIL_WG * NW rows on (NW: the kernel's waves a workgroup). The held rows: the plan's span, or where it
// records none, the rows' owners in row_info.
constexpr int PF_TAIL_WG = 256;
template <int NW> __device__ __forceinline__ void zero_dead_rows(const Exl3c4Launch& a, int z) {
    const int lane = threadIdx.x & 63;
    const bool span = a.plan[EXL3C4_PF_SPAN] != 0;
    const int lo = a.plan[EXL3C4_PF_SPAN + 1], hi = a.plan[EXL3C4_PF_SPAN + 2];
    for (int64_t i = (int64_t)z * NW + (threadIdx.x >> 6); i < a.T; i += (int64_t)PF_TAIL_WG * NW) {
        if (span ? (i >= lo && i < hi) : a.row_info[2 * i] >= 0) continue;   // held: a chunk writes it
        uint16_t* out = (uint16_t*)a.y + i * a.y_pitch;
        for (int b = 0; b < a.nblk; ++b) {
            out[b * 128 + lane] = 0;
            out[b * 128 + lane + 64] = 0;
        }
    }
}

// The staged input of one 64-k step of a chunk of R = 16 NT rows: R rows x 4 groups of 16 halves, a group two 16-byte
// loads, spread over 256 threads (H = ceil(R / 64) groups a thread; a slot past the R x 4 groups reloads the last one,
// so that the loads stay unconditional and their waits exact). Rows past the chunk load a copy of its last row. A
// slot's address is the step's base (wave-uniform: scalar registers) plus the slot's byte offset, fixed for the chunk
// and held in a register (32 bits: 2 q pitch + 48 < 2^32 for the q < 96 rows of a chunk, which the host's choice of
// the prefill path keeps), so the steps' loads take no address arithmetic. The groups land in LDS in row order, k in
// order: pf_step pairs the decoded B registers to match.
template <int NT> struct StageRegs {
    static constexpr int H = (NT + 3) / 4;                        // slots a thread
    u32x4_t v[2 * H];
    uint32_t off[H];                                              // each slot's byte offset from the step's base
};
template <int NT>
__device__ __forceinline__ void stage_init(int64_t pitch, int nrows, StageRegs<NT>& r, int tid) {
    constexpr int G = 64 * NT;                                    // groups a step
#pragma unroll
    for (int h = 0; h < StageRegs<NT>::H; ++h) {
        const int g = min(tid + 256 * h, G - 1);
        const uint32_t q = (uint32_t)min(g >> 2, nrows - 1), grp = (uint32_t)(g & 3);
        r.off[h] = (q * (uint32_t)pitch + grp * 16u) * 2u;
    }
}
// base: the step's first staged column of the chunk's first row, wave-uniform
template <int NT> __device__ __forceinline__ void stage_load(const uint16_t* base, StageRegs<NT>& r) {
#pragma unroll
    for (int h = 0; h < StageRegs<NT>::H; ++h) {
        const __attribute__((address_space(1))) u32x4_t* p = (const __attribute__((address_space(1))) u32x4_t*)
            ((const __attribute__((address_space(1))) char*)base + (uint64_t)r.off[h]);
        r.v[2 * h] = p[0];
        r.v[2 * h + 1] = p[1];
    }
}
// ... and its store into a step buffer [R][kp]
template <int NT>
__device__ __forceinline__ void stage_store(uint16_t* A, int kp, const StageRegs<NT>& r, int tid) {
    constexpr int G = 64 * NT;
#pragma unroll
    for (int h = 0; h < StageRegs<NT>::H; ++h) {
        const int g = tid + 256 * h;
        if (g >= G) break;                                        // uniform in a wave (G is a multiple of 64)
        const int q = g >> 2, grp = g & 3;
        u32x4_t* d = (u32x4_t*)(A + q * kp + grp * 16);
        d[0] = r.v[2 * h];
        d[1] = r.v[2 * h + 1];
    }
}

// The prefill GEMMs' workgroups and XCDs: XCD x (the dispatcher deals linear ids g to the XCDs in turn, x = g % 8)
// takes the plan's contiguous chunk range [xb[x], xb[x + 1]) -- ranges of about equal cost, from k_plan -- as
// n = per x (its chunks) units in this GEMM's order (ord: the chunks of more row tiles first, so the range's last
// units are its shortest; unit s: the (s % per)-th running unit -- column group or block -- of the range's (s /
// per)-th chunk). Slot g / 8 takes unit g / 8 itself, up to the range's last R units; those are dealt by the XCD's
// cursor (cur + 32 x, zeroed by the plan) to its later slots, and a slot that finds its XCD's cursor spent takes one
// from the XCD with the most units left (a range's cost is an estimate: the XCDs' ends spread by about half a unit),
// or returns false when every range is spent. A chunk's units run side by side in one L2, so its staged rows come
// from HBM once; an expert's chunks fall in one or two ranges, its full chunks side by side in one tile class, so
// they too share an L2 and, running close in time, read the expert's codes from HBM about once. No workgroup waits;
// the cursors hand out each unit once, and the grid's pf_xcd_bound chunks' units an XCD cover every range. (Where a
// workgroup lands changes no bits.)
template <int R>
__device__ __forceinline__ bool xcd_unit(int per, const int32_t* xb, const int32_t* ord, int32_t* cur, int& unit,
                                         int& chunk) {
    const int g = (int)blockIdx.x, slot = g >> 3, x = g & 7;
    const int n = (xb[x + 1] - xb[x]) * per, st = max(n - R, 0);
    if (slot >= n + R) return false;                              // past the range's end by a round: nothing to take
    int y = x, s = slot;
    if (slot >= st) {                                             // the range's last R units, or R slots past its end
        __shared__ int take_s[2];
        if (threadIdx.x == 0) {
            int ty = -1, ts = 0;
            if (slot < n) {                                       // a slot of the range: its cursor first
                const int v = st + __hip_atomic_fetch_add(cur + 32 * x, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (v < n) {
                    ty = x;
                    ts = v;
                }
            }
            // past the range (the first R of the grid's slots beyond it), or its cursor spent: the XCD with the most
            // units left.
            // Each failed take finds a range spent that the next search skips, so 8 searches see every range spent.
            for (int tries = 0; ty < 0 && tries < 8; ++tries) {
                int best = -1, left = 0, lz[8];
#pragma unroll
                for (int z = 0; z < 8; ++z)
                    lz[z] = __hip_atomic_load(cur + 32 * z, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#pragma unroll
                for (int z = 0; z < 8; ++z) {
                    const int nz = (xb[z + 1] - xb[z]) * per, rz = nz - max(nz - R, 0) - lz[z];
                    if (rz > left) {
                        left = rz;
                        best = z;
                    }
                }
                if (best < 0) break;
                const int nb = (xb[best + 1] - xb[best]) * per, sb = max(nb - R, 0);
                const int v = sb + __hip_atomic_fetch_add(cur + 32 * best, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                if (v < nb) {
                    ty = best;
                    ts = v;
                }
            }
            take_s[0] = ty;
            take_s[1] = ts;
        }
        __syncthreads();
        y = take_s[0];
        s = take_s[1];
        if (y < 0) return false;
    }
    const int q = s / per;
    unit = s - q * per;
    chunk = ord[xb[y] + q];
    return true;
}
// each XCD's units dealt by its cursor: gate_up's last round of its slots (2 workgroups a CU x 32 CUs); down's none
// -- its XCDs end within a few us, and a round dealt by cursors (128 units) measured 2 us slower than static slots
constexpr int PF_DYN_GU = 64, PF_DYN_DN = 0;

// One k-step of the prefill GEMM: the step's B operands (decoded just before) against each of the chunk's NT row
// tiles (4 MFMAs a tile), each group ending in mfma_guard: gfx950 does not interlock a VALU or LDS write against an
// in-flight 16x16x32 MFMA's A/B reads, and the compiler does not pad for it. (A step's decode and its MFMAs take
// their sum on a SIMD of 4 such waves, measured: the decode keeps the VALU pipe full and the MFMAs of the other waves
// find no slot beside it; a step issued behind the next step's decode, or the waves split into a decoding and a
// multiplying half each half-step, gained nothing.)
constexpr int PF_NT = EXL3C4_PF_ROWS / 16;                      // a chunk's row tiles at most
// a chunk's row tiles at most at K = BITS (pf_rows: seven where the launch's K are at most 4)
template <int BITS> constexpr int pf_nt() { return BITS <= 4 ? EXL3C4_PF_ROWS / 16 : EXL3C4_PF_ROWS_WIDE / 16; }
template <int BITS, int CB, int NT>
__device__ __forceinline__ void pf_step(const uint16_t* Ab, int kp, const uint32_t (&B)[16], float4_t (&acc)[PF_NT][2]) {
    // the segment's B[j] holds the k pair 2 j' of the lane's 16-group for j' = (0, 4, 1, 5, 2, 6, 3, 7)[j & 7] (the
    // trellis segment's run order); the staged group is in k order, so Aa (k 0..7) pairs with B[0, 2, 4, 6] and
    // Ac (k 8..15) with B[1, 3, 5, 7] (and the second 16 columns' with B[8..15] alike)
    const half8_t b0 = as_half8(B[0], B[2], B[4], B[6]), b1 = as_half8(B[8], B[10], B[12], B[14]);
    const half8_t b2 = as_half8(B[1], B[3], B[5], B[7]), b3 = as_half8(B[9], B[11], B[13], B[15]);
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        const uint16_t* arow = Ab + t * 16 * kp;
        const half8_t Aa = *(const half8_t*)arow, Ac = *(const half8_t*)(arow + 8);
        acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Aa, b0, acc[t][0], 0, 0, 0);
        acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Aa, b1, acc[t][1], 0, 0, 0);
        acc[t][0] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ac, b2, acc[t][0], 0, 0, 0);
        acc[t][1] = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ac, b3, acc[t][1], 0, 0, 0);
        mfma_guard(Aa, Ac, b0, b1, b2, b3);
    }
}

// The prefill GEMM of one chunk (<= EXL3C4_PF_ROWS rows of one expert) against the strips of one workgroup, all of k:
// the input streams through two LDS step buffers (64 k each, a half at a time), the next step's loads in flight while
// this one is multiplied; each wave decodes its strip's step once and runs it against every row tile (pf_step). NH = 1:
// 4 waves, one staged input (columns col_off + k). NH = 2: 8 waves, two staged inputs (columns k and half_off + k),
// thread t staging half t / 256 and wave w reading half w / 4. NT: the chunk's 16-row tiles (ceil(nrows / 16)), a
// template argument so that the loop holds no branch on it and stages only the rows it has. Accumulations:
// acc[row tile][strip half]. The weight: entry jx of the codes table (codes, codes_s) of k = KC columns.
constexpr int PF_KP = EXL3C4_KSTEP + 8;                           // a staged row, padded: 16 rows hit 16 bank groups
template <int BITS, int CB, int NH, int NT>
__device__ __forceinline__ void pf_gemm_nt(const void* codes, int32_t codes_s, int KC, int64_t jx, int strip,
                                        const uint16_t* src, int64_t pitch, int row0, int nrows, int col_off,
                                        int half_off, uint16_t* lds, float4_t (&acc)[PF_NT][2]) {
    const int lane = threadIdx.x & 63;
    const int nb = KC / 128, ksteps = KC / EXL3C4_KSTEP;
    constexpr int kp = PF_KP;
#pragma unroll
    for (int t = 0; t < NT; ++t) acc[t][0] = acc[t][1] = float4_t{ 0.f, 0.f, 0.f, 0.f };   // the chunk's tiles only
    const int tid = (int)threadIdx.x & 255;
    const int sh = NH == 2 ? __builtin_amdgcn_readfirstlane((int)threadIdx.x >> 8) : 0;   // staged and read half
    const uint16_t* sbase = src + (int64_t)row0 * pitch + col_off + sh * half_off;   // wave-uniform
    auto bufp = [&](int b, int h) { return lds + (b * NH + h) * EXL3C4_PF_ROWS * kp; };
    const gu32p rec = (gu32p)tab_entry(codes, codes_s, jx) + (int64_t)strip * ksteps * 64 * BITS + lane * BITS;
    // the codes of the steps ahead: dA even steps, dB odd; each refill 2 steps ahead of the step it serves (clamped:
    // past the stream a harmless reload of the last step, unconditional so that the waits count exactly)
    uint32_t dA[BITS], dB[BITS];
    load_words<BITS>(rec, dA);
    load_words<BITS>(rec + 64 * BITS, dB);
    StageRegs<NT> r;
    stage_init<NT>(pitch, nrows, r, tid);
    stage_load<NT>(sbase, r);
    const Mul1Consts k = mul1_consts();
    stage_store<NT>(bufp(0, sh), kp, r, tid);
    __syncthreads();
    const int rr = lane & 15, g = lane >> 4;
    int kb = 0;
    do {                                                          // nb >= 1: the launch checks refuse k of 0
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {                          // step ks = 2 kb + s2 sits in buffer s2
            const int ks = 2 * kb + s2;
            // the next step, or at the last a harmless reload of it: unconditional, like the codes' refills
            stage_load<NT>(sbase + min(ks + 1, ksteps - 1) * EXL3C4_KSTEP, r);
            uint32_t B[16];
            decode_segment<BITS, CB>(s2 ? dB : dA, B, k);
            const int nx = min(ks + 2, ksteps - 1);
            if (s2 == 0) load_words<BITS>(rec + (int64_t)nx * 64 * BITS, dA);
            else load_words<BITS>(rec + (int64_t)nx * 64 * BITS, dB);
            pf_step<BITS, CB, NT>(bufp(s2, sh) + rr * kp + 16 * g, kp, B, acc);
            if (ks + 1 < ksteps) stage_store<NT>(bufp(s2 ^ 1, sh), kp, r, tid);
            __syncthreads();
        }
    } while (++kb < nb);
}

template <int BITS, int CB, int NH>
__device__ __forceinline__ void pf_gemm(const void* codes, int32_t codes_s, int KC, int64_t jx, int strip,
                                        const uint16_t* src, int64_t pitch, int row0, int nrows, int col_off,
                                        int half_off, uint16_t* lds, float4_t (&acc)[PF_NT][2]) {
#define EXL3C4_PF_ARGS codes, codes_s, KC, jx, strip, src, pitch, row0, nrows, col_off, half_off, lds, acc
    static_assert(PF_NT == 7, "pf_gemm instantiates 1 to 7 row tiles");
    const int nt = (nrows + 15) >> 4;                             // at most pf_nt<BITS>: the plan's pf_rows
    if constexpr (pf_nt<BITS>() == 7) {
        if (nt >= 7) {
            pf_gemm_nt<BITS, CB, NH, 7>(EXL3C4_PF_ARGS);
            return;
        }
    }
    switch (nt) {
    case 1: pf_gemm_nt<BITS, CB, NH, 1>(EXL3C4_PF_ARGS); break;
    case 2: pf_gemm_nt<BITS, CB, NH, 2>(EXL3C4_PF_ARGS); break;
    case 3: pf_gemm_nt<BITS, CB, NH, 3>(EXL3C4_PF_ARGS); break;
    case 4: pf_gemm_nt<BITS, CB, NH, 4>(EXL3C4_PF_ARGS); break;
    case 5: pf_gemm_nt<BITS, CB, NH, 5>(EXL3C4_PF_ARGS); break;
    default: pf_gemm_nt<BITS, CB, NH, 6>(EXL3C4_PF_ARGS); break;
    }
#undef EXL3C4_PF_ARGS
}

// gate_up's prefill GEMM with its epilogue: one workgroup of 8 waves per (chunk, h-block hb): waves 0..3 the 4 gate
// strips of columns 128 hb .., waves 4..7 the 4 up strips of columns N / 2 + 128 hb .., each half of xr staged for
// its waves. With keep_sums the raw sums go to part (a checker's view). Then the accumulations cross LDS and each
// wave finishes whole rows of the block: had128, x svh, f16(silu(gate) * up), and with h_rot down's first step
// f16(had(f16(h * dn_suh))) (kernels/exl3ref/ref.c:187-212) into y at columns 128 hb... A negative sorted_tok, and a
// narrower class's blocks past its width, are written zero; rows no run holds are the tail workgroups'.
template <int BITS, int CB>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_gu_pf(const Exl3c4Launch a) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * 2 * EXL3C4_PF_ROWS * PF_KP];
    constexpr int ACC_PITCH = 264;                                // floats: the epilogue's [48][256] with padding
    constexpr int EPI_T = 3;                                      // row tiles an epilogue pass (48 rows)
    static_assert(EPI_T * 16 * ACC_PITCH * 4 <= (int)sizeof(lds), "an epilogue pass fits the staging buffers");
    if (a.tail_from && (int)blockIdx.x >= a.tail_from) {          // gate_up alone: the rows no run holds
        zero_dead_rows<8>(a, (int)blockIdx.x - a.tail_from);
        return;
    }
    int hb, chunk;
    if (!xcd_unit<PF_DYN_GU>(a.n_grp / 2, a.plan + EXL3C4_PF_XCD_GU, pf_order(a, 0), a.plan + EXL3C4_PF_CUR, hb,
                             chunk))
        return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int4 ent = ((const int4*)(a.plan + EXL3C4_PF_PLAN_HDR))[chunk];
    const int e = __builtin_amdgcn_readfirstlane(ent.x), row0 = __builtin_amdgcn_readfirstlane(ent.y),
              nrows = __builtin_amdgcn_readfirstlane(ent.z);      // one chunk a workgroup: uniform
    const Exl3c4DevClass& K = a.cls[class_of(a, e)];
    const int64_t jx = entry_of(a, e);
    const int N = K.rows, KC = K.cols, width = N / 2;
    if (hb * 128 >= width) {                                      // a narrower class: its rows' block past its width
        if (hb < a.nblk)
            for (int q = wave; q < nrows; q += 8) {
                uint16_t* out = (uint16_t*)a.y + (int64_t)(row0 + q) * a.y_pitch + hb * 128;
                out[lane] = 0;
                out[lane + 64] = 0;
            }
        return;
    }
    const int half = wave >> 2, strip = half ? N / 64 + 4 * hb + (wave & 3) : 4 * hb + wave;
    // the chunk's sorted_tok, lane q holding row q (srt) and row 64 + q (srt2), taken by readlane
    const int srt = a.sorted[row0 + min(lane, nrows - 1)], srt2 = a.sorted[row0 + min(64 + lane, nrows - 1)];
    float4_t acc[PF_NT][2];                                       // pf_gemm zeroes the chunk's tiles
    pf_gemm<BITS, CB, 2>(K.codes, K.codes_s, KC, jx, strip, (const uint16_t*)a.x, a.x_pitch, row0, nrows, 0, KC, lds,
                         acc);
    const int cc = lane & 15, rg = lane >> 4;
    const int n = strip * EXL3C4_STRIP + 16 * (cc & 1) + (cc >> 1);
    const int col_l = half * 128 + (wave & 3) * EXL3C4_STRIP + 16 * (cc & 1) + (cc >> 1);
    // The epilogue in had128_x8's layout: the accumulations cross LDS EPI_T row tiles at a time, then the waves take
    // the pass's rows four at a time, a 16-lane row of the wave per row, lane l holding the 8 consecutive columns
    // 8 g .. 8 g + 7 of the block (g = rot_group(l & 15)) of gate and of up: had128, x svh, f16(silu(gate) * up), and
    // with h_rot f16(had(f16(h * dn_suh))), the reference's steps and roundings (gate_up_math's, in another lane
    // layout), then one 16-byte store a lane.
    const int g = rot_group(lane & 15), gcol = hb * 128 + 8 * g;  // the lane's first column of the block
    const RotSigns ks = rot_signs(g);
    uint32_t sg[4], su[4], sd[4];                                 // svh (gate, up) and dn_suh of those columns
    {
        const uint16_t* svh = (const uint16_t*)tab_entry(K.svh, K.svh_s, jx);
        const bool sw = (((uintptr_t)svh) & 15) == 0 && (width & 7) == 0;
        load8w(svh + gcol, sw, sg);
        load8w(svh + width + gcol, sw, su);
        if (a.h_rot) {
            const uint16_t* ds = (const uint16_t*)tab_entry(K.dn_suh, K.dn_suh_s, jx);
            load8w(ds + gcol, (((uintptr_t)ds) & 15) == 0, sd);
        } else {
            sd[0] = sd[1] = sd[2] = sd[3] = 0;
        }
    }
    float sgf[8], suf[8];                                         // the gate and up scales as f32, once
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        sgf[j] = h2f((uint16_t)(sg[j >> 1] >> (16 * (j & 1))));
        suf[j] = h2f((uint16_t)(su[j >> 1] >> (16 * (j & 1))));
    }
    const bool yw = ((((uintptr_t)a.y) | ((uintptr_t)a.y_pitch * 2)) & 15) == 0;
    float* acc_l = (float*)lds;                                   // [48][ACC_PITCH], over the staging buffers
#pragma unroll
    for (int p = 0; p < (pf_nt<BITS>() + EPI_T - 1) / EPI_T; ++p) {   // the last pass may hold fewer tiles
        const int r0 = p * EPI_T * 16;                            // the pass's first chunk row
        if (r0 >= nrows) break;                                   // uniform
        if (p) __syncthreads();                                   // the previous pass's rows are read
#pragma unroll
        for (int tt = 0; tt < EPI_T; ++tt)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int t = p * EPI_T + tt, row = t * 16 + rg * 4 + q;
                if (t < pf_nt<BITS>() && row < nrows) {
                    if (a.keep_sums) {
                        a.part[(int64_t)(row0 + row) * a.part_pitch + n] = acc[t][0][q];
                        a.part[(int64_t)(row0 + row) * a.part_pitch + n + 8] = acc[t][1][q];
                    }
                    acc_l[(row - r0) * ACC_PITCH + col_l] = acc[t][0][q];
                    acc_l[(row - r0) * ACC_PITCH + col_l + 8] = acc[t][1][q];
                }
            }
        __syncthreads();
        const int rend = min(nrows, r0 + EPI_T * 16);
        for (int rb = r0 + 4 * wave; rb < rend; rb += 32) {       // uniform: the wave's four rows start in the pass
            const int row = rb + (lane >> 4);                     // rows past the pass: computed, not stored
            const float* pp = acc_l + (min(row, r0 + EPI_T * 16 - 1) - r0) * ACC_PITCH + 8 * g;
            const float4_t g_lo = *(const float4_t*)pp, g_hi = *(const float4_t*)(pp + 4);
            const float4_t u_lo = *(const float4_t*)(pp + 128), u_hi = *(const float4_t*)(pp + 132);
            float gv[8] = { g_lo[0], g_lo[1], g_lo[2], g_lo[3], g_hi[0], g_hi[1], g_hi[2], g_hi[3] };
            float uv[8] = { u_lo[0], u_lo[1], u_lo[2], u_lo[3], u_hi[0], u_hi[1], u_hi[2], u_hi[3] };
            const int tk_lo = __shfl(srt, row & 63), tk_hi = __shfl(srt2, row & 63);
            const int tk = row < 64 ? tk_lo : tk_hi;
            had128_x8(gv, ks);
            had128_x8(uv, ks);
            uint32_t o[4];                                        // h, two f16 values a dword
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const float h0 = silu(gv[2 * j] * sgf[2 * j]) * (uv[2 * j] * suf[2 * j]);
                const float h1 = silu(gv[2 * j + 1] * sgf[2 * j + 1]) * (uv[2 * j + 1] * suf[2 * j + 1]);
                o[j] = f2h2(h0, h1);
            }
            if (a.h_rot) {
                // f16(h dn_suh): one f16 multiply of the pair (the exact product rounded once, as f16(f32 f32) rounds
                // it), its first butterfly stage straight from the packed product (mix_sum_diff), then the rest
                float rv[8];
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const half2_t pr = __builtin_bit_cast(half2_t, o[j]) * __builtin_bit_cast(half2_t, sd[j]);
                    mix_sum_diff(__builtin_bit_cast(uint32_t, pr), rv[2 * j], rv[2 * j + 1]);
                }
                had128_x8<2>(rv, ks);
#pragma unroll
                for (int j = 0; j < 4; ++j) o[j] = f2h2(rv[2 * j], rv[2 * j + 1]);
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = tk < 0 ? 0u : o[j];
            if (row < rend) {
                uint16_t* out = (uint16_t*)a.y + (int64_t)(row0 + row) * a.y_pitch + gcol;
                if (yw) {
                    *(uint4*)out = uint4{ o[0], o[1], o[2], o[3] };
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        out[2 * j] = (uint16_t)o[j];
                        out[2 * j + 1] = (uint16_t)(o[j] >> 16);
                    }
                }
            }
        }
    }
}

// down's prefill GEMM: one workgroup per (chunk, 128-column output block); h (rotated, sorted-row order) in; the
// epilogue (had128, x svh, bf16) in the workgroup through LDS, one row tile at a time. Writes every row of its chunk
// in its block: a negative sorted_tok and a narrower class's tail as zero; with keep_sums the raw sums to dacc.
template <int BITS, int CB>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4, 8))) void k_dn_pf(const Exl3c4Launch a) {
    __shared__ __attribute__((aligned(16))) uint16_t lds[2 * EXL3C4_PF_ROWS * PF_KP];
    if (a.tail_from && (int)blockIdx.x >= a.tail_from) {          // the rows no run holds
        zero_dead_rows<4>(a, (int)blockIdx.x - a.tail_from);
        return;
    }
    int b, chunk;
    if (!xcd_unit<PF_DYN_DN>(a.nblk, a.plan + EXL3C4_PF_XCD_DN, pf_order(a, 1), a.plan + EXL3C4_PF_CUR + 256, b,
                             chunk))
        return;
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int4 ent = ((const int4*)(a.plan + EXL3C4_PF_PLAN_HDR))[chunk];
    const int e = __builtin_amdgcn_readfirstlane(ent.x), row0 = __builtin_amdgcn_readfirstlane(ent.y),
              nrows = __builtin_amdgcn_readfirstlane(ent.z);      // one chunk a workgroup: uniform
    const DnW D = dn_weight(a.dn_gd, a.cls[class_of(a, e)]);
    const int64_t jx = entry_of(a, e);
    const int N = D.rows;
    if (b * 128 >= N) {                                           // a narrower class's tail
        for (int q = wave; q < nrows; q += 4) {
            uint16_t* out = (uint16_t*)a.y + (int64_t)(row0 + q) * a.y_pitch + b * 128;
            out[lane] = 0;
            out[lane + 64] = 0;
        }
        return;
    }
    float4_t acc[PF_NT][2];                                       // pf_gemm zeroes the chunk's tiles
    pf_gemm<BITS, CB, 1>(D.codes, D.codes_s, D.cols, jx, 4 * b + wave, (const uint16_t*)a.x, a.x_pitch, row0, nrows, 0, 0,
                         lds, acc);
    // the chunk's sorted_tok, lane q holding row q (srt) and row 64 + q (srt2), taken by readlane: loaded after the
    // GEMM, so that at K <= 4 the loop's seven row tiles of accumulators fit 4 waves a SIMD without a spill
    const int srt = a.sorted[row0 + min(lane, nrows - 1)], srt2 = a.sorted[row0 + min(64 + lane, nrows - 1)];

    // The epilogue, a tile's 16 rows at a time: the sums cross LDS, then wave w takes the tile's rows 4 w .. 4 w + 3,
    // a 16-lane row of the wave per row, lane l holding the 8 consecutive columns 8 g .. 8 g + 7 of the block
    // (g = rot_group(l & 15)) -- had128_x8's layout: its stages h = 1, 2, 4 inside the lane, h = 8 .. 64 one DPP
    // v_fmac each within the 16-lane row -- then x svh, bf16, and one 16-byte store a lane.
    const void* svh = tab_entry(D.svh, D.svh_s, jx);
    const int g = rot_group(lane & 15), gcol = b * 128 + 8 * g;   // the lane's first column in y
    const RotSigns ks = rot_signs(g);
    float sv[8];
    {
        uint32_t s4[4];
        load8w((const uint16_t*)svh + gcol, (((uintptr_t)svh) & 15) == 0, s4);
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            sv[2 * j] = h2f((uint16_t)s4[j]);
            sv[2 * j + 1] = h2f((uint16_t)(s4[j] >> 16));
        }
    }
    const bool yw = ((((uintptr_t)a.y) | ((uintptr_t)a.y_pitch * 2)) & 15) == 0;
    constexpr int EP = 132;                                       // floats a staged row: 16-byte rows off one bank
    float* acc_l = (float*)lds;                                   // [16][EP], one row tile at a time
    const int cc = lane & 15, rg = lane >> 4;
    const int col = 32 * wave + 16 * (cc & 1) + (cc >> 1);
    const int ntile = (nrows + 15) >> 4;
    const int lrow = 4 * wave + (lane >> 4);                      // this lane's row of a tile
#pragma unroll
    for (int t = 0; t < pf_nt<BITS>(); ++t) {                     // unrolled: acc[t] stays in registers
        if (t >= ntile) break;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc_l[(rg * 4 + q) * EP + col] = acc[t][0][q];
            acc_l[(rg * 4 + q) * EP + col + 8] = acc[t][1][q];
        }
        __syncthreads();
        if (t * 16 + 4 * wave < nrows) {                          // uniform: the wave holds a row of the chunk
            const int row = t * 16 + lrow;                        // rows past the chunk: computed, not stored
            const float4_t lo = *(const float4_t*)(acc_l + lrow * EP + 8 * g);
            const float4_t hi = *(const float4_t*)(acc_l + lrow * EP + 8 * g + 4);
            float v[8] = { lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3] };
            const int tk_lo = __shfl(srt, row & 63), tk_hi = __shfl(srt2, row & 63);
            const int tk = row < 64 ? tk_lo : tk_hi;
            had128_x8(v, ks);
            uint32_t o[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) o[j] = tk < 0 ? 0u : f2bf2(v[2 * j] * sv[2 * j], v[2 * j + 1] * sv[2 * j + 1]);
            if (row < nrows) {
                const int64_t r = row0 + row;
                if (a.keep_sums) {
                    float* dacc = a.dacc + r * a.dacc_pitch + gcol;
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        dacc[j] = lo[j];
                        dacc[4 + j] = hi[j];
                    }
                }
                uint16_t* out = (uint16_t*)a.y + r * a.y_pitch + gcol;
                if (yw) {
                    *(uint4*)out = uint4{ o[0], o[1], o[2], o[3] };
                } else {
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        out[2 * j] = (uint16_t)o[j];
                        out[2 * j + 1] = (uint16_t)(o[j] >> 16);
                    }
                }
            }
        }
        __syncthreads();
    }
}

// dequant: one wave per block of the stored record; W_hat[n][k] fp16 bits, the radiance [rows, cols] view.
template <int BITS, int CB>
__global__ __launch_bounds__(256) void k_dequant(const uint32_t* rec, int rows, int cols, uint16_t* w, int64_t pitch) {
    const int lane = threadIdx.x & 63;
    const int64_t blk = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int ksteps = cols / EXL3C4_KSTEP, strips = rows / EXL3C4_STRIP;
    if (blk >= (int64_t)ksteps * strips) return;
    const int strip = (int)(blk / ksteps), ks = (int)(blk % ksteps);
    uint32_t d[BITS];
    load_words<BITS>((const __attribute__((address_space(1))) uint32_t*)rec + (blk * 64 + lane) * BITS, d);
    uint32_t B[16];
    decode_segment<BITS, CB>(d, B, mul1_consts());
    const int cc = lane & 15, g = lane >> 4;
    const int n0 = strip * EXL3C4_STRIP + 16 * (cc & 1) + (cc >> 1), k0 = ks * EXL3C4_KSTEP + 16 * g;
#pragma unroll
    for (int R = 0; R < 4; ++R)
#pragma unroll
        for (int jp = 0; jp < 8; ++jp) {
            const int l = 2 * (R & 1) + (jp >> 2), jj = jp & 3;
            const int k = k0 + 2 * l + ((jj & 1) | ((jj & 2) << 2));
            const int n = n0 + 8 * (R >> 1);
            const uint32_t word = B[R * 4 + (jp >> 1)];
            w[(int64_t)n * pitch + k] = (uint16_t)((jp & 1) ? (word >> 16) : (word & 0xFFFFu));
        }
}

// ------------------------------------------------------------------------------------------------ dispatch

typedef void (*GemmFn)(const Exl3c4Launch);
typedef void (*DequantFn)(const uint32_t*, int, int, uint16_t*, int64_t);

template <template <int, int> class F, int BITS> GemmFn by_cb(int cb) {
    switch (cb) {
    case EXL3C4_CB_MUL1: return F<BITS, EXL3C4_CB_MUL1>::fn;
    case EXL3C4_CB_MCG:  return F<BITS, EXL3C4_CB_MCG>::fn;
    default:             return F<BITS, EXL3C4_CB_3INST>::fn;
    }
}
template <template <int, int> class F> GemmFn by_bits(int bits, int cb) {
    switch (bits) {
    case 2: return by_cb<F, 2>(cb);
    case 3: return by_cb<F, 3>(cb);
    case 4: return by_cb<F, 4>(cb);
    case 5: return by_cb<F, 5>(cb);
    case 6: return by_cb<F, 6>(cb);
    case 7: return by_cb<F, 7>(cb);
    case 8: return by_cb<F, 8>(cb);
    default: return nullptr;
    }
}
template <int BITS, int CB> struct GuK { static constexpr GemmFn fn = k_gu<BITS, CB>; };
template <int BITS, int CB> struct DnK { static constexpr GemmFn fn = k_dn<BITS, CB>; };
template <int BITS, int CB> struct GdK { static constexpr GemmFn fn = k_gd<BITS, CB>; };
template <int BITS, int CB> struct GuPfK { static constexpr GemmFn fn = k_gu_pf<BITS, CB>; };
template <int BITS, int CB> struct DnPfK { static constexpr GemmFn fn = k_dn_pf<BITS, CB>; };

template <int BITS> DequantFn dequant_fn(int cb) {
    switch (cb) {
    case EXL3C4_CB_MUL1: return k_dequant<BITS, EXL3C4_CB_MUL1>;
    case EXL3C4_CB_MCG:  return k_dequant<BITS, EXL3C4_CB_MCG>;
    default:             return k_dequant<BITS, EXL3C4_CB_3INST>;
    }
}
DequantFn pick_dequant(int bits, int cb) {
    switch (bits) {
    case 1: return dequant_fn<1>(cb);
    case 2: return dequant_fn<2>(cb);
    case 3: return dequant_fn<3>(cb);
    case 4: return dequant_fn<4>(cb);
    case 5: return dequant_fn<5>(cb);
    case 6: return dequant_fn<6>(cb);
    case 7: return dequant_fn<7>(cb);
    case 8: return dequant_fn<8>(cb);
    default: return nullptr;
    }
}

int launched(void) { return hipGetLastError() == hipSuccess ? 0 : EXL3C4_E_DEVICE; }

// A plain launch, or one whose dispatch stamps two events at its own start and end (the timing of one kernel).
template <typename F, typename... Args>
int go(F f, unsigned blocks, hipStream_t s, void* ev0, void* ev1, Args... args) {
    if (ev0 && ev1)
        hipExtLaunchKernelGGL(f, dim3(blocks), dim3(256), 0, s, (hipEvent_t)ev0, (hipEvent_t)ev1, 0, args...);
    else
        hipLaunchKernelGGL(f, dim3(blocks), dim3(256), 0, s, args...);
    return launched();
}

unsigned blocks_for_waves(int64_t waves) { return (unsigned)((waves + 3) / 4); }

template <typename F, typename... Args>
int go2(F f, dim3 grid, hipStream_t s, void* ev0, void* ev1, uint32_t lds, Args... args) {
    if (ev0 && ev1)
        hipExtLaunchKernelGGL(f, grid, dim3(256), lds, s, (hipEvent_t)ev0, (hipEvent_t)ev1, 0, args...);
    else
        hipLaunchKernelGGL(f, grid, dim3(256), lds, s, args...);
    return hipGetLastError() == hipSuccess ? 0 : EXL3C4_E_DEVICE;
}

// down's LDS: the staged rows [chunk_rows][lds_pitch] halves, later the block's accumulations [chunk_rows][128] f32
// over them
uint32_t dn_lds_bytes(const Exl3c4Launch* a) {
    const uint32_t rows = (uint32_t)(a->chunk_rows * a->lds_pitch * 2), acc = (uint32_t)(a->chunk_rows * 128 * 4);
    return rows > acc ? rows : acc;
}

}  // namespace

extern "C" int exl3c4_dev_prep(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    const int64_t waves = (int64_t)a->T * 2 * (a->x_cols_max / 128);
    if (waves <= 0) return 0;
    return go(k_prep, blocks_for_waves(waves), (hipStream_t)stream, ev0, ev1, *a);
}

extern "C" int exl3c4_dev_gu(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    const GemmFn f = by_bits<GuK>(a->bits, a->codebook);
    if (!f) return EXL3C4_E_DTYPE;
    if (a->T <= 0 || a->n_grp <= 0) return 0;
    const uint32_t lds = (uint32_t)(a->chunk_rows * a->lds_pitch * 2);
    return go2(f, dim3((unsigned)(a->n_grp * a->ksplit), (unsigned)a->T), (hipStream_t)stream, ev0, ev1, lds, *a);
}

extern "C" int exl3c4_dev_gepi(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    const int per = a->blk_per_wave > 0 ? a->blk_per_wave : 1;
    const int64_t waves = (int64_t)a->T * ((a->nblk + per - 1) / per);
    if (waves <= 0) return 0;
    if (a->ksplit >= 8) return go(k_gepi<8>, blocks_for_waves(waves), (hipStream_t)stream, ev0, ev1, *a);
    return go(k_gepi<4>, blocks_for_waves(waves), (hipStream_t)stream, ev0, ev1, *a);
}

extern "C" int exl3c4_dev_dn(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    const GemmFn f = by_bits<DnK>(a->dn_gd ? a->dn_bits : a->bits, a->codebook);
    if (!f) return EXL3C4_E_DTYPE;
    if (a->nblk <= 0 || a->T <= 0) return 0;
    return go2(f, dim3((unsigned)a->nblk, (unsigned)a->T), (hipStream_t)stream, ev0, ev1, dn_lds_bytes(a), *a);
}

// gate_up_down's kernel for gate_up's K and down's: the same K for every codebook, a mixed pair for mul1 (2..8 each)
template <int BG, int BD> GemmFn gd_mixed_bd() { return k_gd<BG, EXL3C4_CB_MUL1, BD>; }
template <int BG> GemmFn gd_mixed(int bd) {
    switch (bd) {
    case 2: return gd_mixed_bd<BG, 2>();
    case 3: return gd_mixed_bd<BG, 3>();
    case 4: return gd_mixed_bd<BG, 4>();
    case 5: return gd_mixed_bd<BG, 5>();
    case 6: return gd_mixed_bd<BG, 6>();
    case 7: return gd_mixed_bd<BG, 7>();
    case 8: return gd_mixed_bd<BG, 8>();
    default: return nullptr;
    }
}
static GemmFn gd_kernel(int bg, int bd, int cb) {
    if (bg == bd) return by_bits<GdK>(bg, cb);
    if (cb != EXL3C4_CB_MUL1) return nullptr;
    switch (bg) {
    case 2: return gd_mixed<2>(bd);
    case 3: return gd_mixed<3>(bd);
    case 4: return gd_mixed<4>(bd);
    case 5: return gd_mixed<5>(bd);
    case 6: return gd_mixed<6>(bd);
    case 7: return gd_mixed<7>(bd);
    case 8: return gd_mixed<8>(bd);
    default: return nullptr;
    }
}

extern "C" int exl3c4_dev_gd(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    const GemmFn f = gd_kernel(a->bits, a->dn_bits, a->codebook);
    if (!f) return EXL3C4_E_DTYPE;
    if (a->T <= 0 || a->n_grp <= 0 || a->nblk <= 0) return 0;
    const uint32_t gu_lds = (uint32_t)(a->chunk_rows * a->lds_pitch_gu * 2), dn_lds = dn_lds_bytes(a);
    const int64_t per_xcd = (int64_t)((a->T + 7) / 8) * (((int64_t)a->n_grp << a->ksplit_log2) + a->nblk) +
                            (a->g_out ? (a->g_ntok + 31) / 32 : 0);  /* gather_empty: 4 tokens a workgroup */
    return go2(f, dim3((unsigned)(8 * per_xcd)), (hipStream_t)stream, ev0, ev1, gu_lds > dn_lds ? gu_lds : dn_lds, *a);
}

// Instance state of the plugin rows (what a row's init hook allocates, never a launch): device memory zeroed once,
// and pinned host memory the device can write (a flag the host reads without a synchronisation).
extern "C" void* exl3c4_dev_zalloc(int64_t bytes) {
    void* p = nullptr;
    if (bytes <= 0 || hipMalloc(&p, (size_t)bytes) != hipSuccess) return nullptr;
    if (hipMemset(p, 0, (size_t)bytes) != hipSuccess || hipDeviceSynchronize() != hipSuccess) {
        (void)hipFree(p);
        return nullptr;
    }
    return p;
}
extern "C" void exl3c4_dev_free(void* p) {
    if (p) (void)hipFree(p);
}
extern "C" void* exl3c4_host_zalloc(int64_t bytes) {
    void* p = nullptr;
    if (bytes <= 0 || hipHostMalloc(&p, (size_t)bytes, hipHostMallocCoherent) != hipSuccess) return nullptr;
    memset(p, 0, (size_t)bytes);
    return p;
}
extern "C" void exl3c4_host_free(void* p) {
    if (p) (void)hipHostFree(p);
}

extern "C" int exl3c4_dev_fill(int32_t* p, int64_t n, void* stream) {
    if (n <= 0) return 0;
    hipLaunchKernelGGL(k_fill, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, (hipStream_t)stream, p, n);
    return launched();
}

extern "C" int exl3c4_dev_plan(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    if (a->T <= 0) return 0;
    if (ev0 && ev1)
        hipExtLaunchKernelGGL(k_plan, dim3(1), dim3(1024), 0, (hipStream_t)stream, (hipEvent_t)ev0, (hipEvent_t)ev1, 0,
                              *a);
    else
        hipLaunchKernelGGL(k_plan, dim3(1), dim3(1024), 0, (hipStream_t)stream, *a);
    return launched();
}

extern "C" int exl3c4_dev_rot(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    if (a->T <= 0) return 0;
    const unsigned nwg = (unsigned)((a->T + 4 * ROT_ROWS - 1) / (4 * ROT_ROWS));
    return go(k_rot, 8 * ((nwg + 7) / 8) + (a->plan ? 1 : 0), (hipStream_t)stream, ev0, ev1, *a);
}

// The most chunks the plan can deal one XCD: the cost midpoints of its chunks lie in a stretch of total / 8 and are
// at least W + 1 apart (each chunk costs W + tiles >= W + 1), so it holds at most total / (8 (W + 1)) + 1 of them;
// total = W x chunks + their tiles <= W max_chunks + pf_tile_budget (the plan keeps no chunk past either).
static int64_t pf_tile_budget(const Exl3c4Launch* a) {
    return (int64_t)a->T / 16 + (a->n_expert < a->T ? a->n_expert : a->T);
}
static int pf_xcd_bound(const Exl3c4Launch* a, int w) {
    return (int)(((int64_t)w * a->max_chunks + pf_tile_budget(a)) / (8 * (w + 1))) + 2;
}

extern "C" int exl3c4_dev_gu_pf(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    const GemmFn f = by_bits<GuPfK>(a->bits, a->codebook);
    if (!f) return EXL3C4_E_DTYPE;
    if (a->n_grp < 2 || a->max_chunks <= 0) return 0;
    Exl3c4Launch g = *a;
    const int units = 8 * (a->n_grp / 2) * pf_xcd_bound(a, EXL3C4_PF_W_GU);
    g.tail_from = a->tail_from ? units : 0;                       // then PF_TAIL_WG workgroups zero dead rows
    const dim3 grid((unsigned)(units + (g.tail_from ? PF_TAIL_WG : 0)));
    if (ev0 && ev1)
        hipExtLaunchKernelGGL(f, grid, dim3(512), 0, (hipStream_t)stream, (hipEvent_t)ev0, (hipEvent_t)ev1, 0, g);
    else
        hipLaunchKernelGGL(f, grid, dim3(512), 0, (hipStream_t)stream, g);
    return launched();
}

extern "C" int exl3c4_dev_dn_pf(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    const GemmFn f = by_bits<DnPfK>(a->dn_gd ? a->dn_bits : a->bits, a->codebook);
    if (!f) return EXL3C4_E_DTYPE;
    if (a->nblk <= 0 || a->max_chunks <= 0) return 0;
    Exl3c4Launch g = *a;
    const int units = 8 * a->nblk * pf_xcd_bound(a, EXL3C4_PF_W_DN);
    g.tail_from = a->tail_from ? units : 0;                       // then PF_TAIL_WG workgroups zero dead rows
    return go2(f, dim3((unsigned)(units + (g.tail_from ? PF_TAIL_WG : 0))), (hipStream_t)stream, ev0, ev1, 0u, g);
}

extern "C" int exl3c4_dev_dequant(const void* record, int32_t rows, int32_t cols, int32_t bits, int32_t codebook,
                                  void* w_hat, int64_t w_pitch, void* stream) {
    const DequantFn f = pick_dequant(bits, codebook);
    if (!f) return EXL3C4_E_DTYPE;
    const int64_t waves = (int64_t)(rows / EXL3C4_STRIP) * (cols / EXL3C4_KSTEP);
    if (waves <= 0) return 0;
    hipLaunchKernelGGL(f, dim3(blocks_for_waves(waves)), dim3(256), 0, (hipStream_t)stream, (const uint32_t*)record,
                       rows, cols, (uint16_t*)w_hat, w_pitch);
    return launched();
}

// The kernels' own narrowing conversions over a list of f32 values (a checker's view): f2bf2 (down's y) on pairs, and
// f2h (h) on each value.
__global__ __launch_bounds__(256) void k_narrow(const float* in, uint16_t* ob, uint16_t* oh, int64_t n) {
    const int64_t j = 2 * ((int64_t)blockIdx.x * 256 + threadIdx.x);
    if (j >= n) return;
    const float lo = in[j], hi = j + 1 < n ? in[j + 1] : 0.f;
    const uint32_t b = f2bf2(lo, hi);
    ob[j] = (uint16_t)b;
    oh[j] = f2h(lo);
    if (j + 1 < n) {
        ob[j + 1] = (uint16_t)(b >> 16);
        oh[j + 1] = f2h(hi);
    }
}

extern "C" int exl3c4_check_narrow(const float* in, uint16_t* out_bf16, uint16_t* out_f16, int64_t n, void* stream) {
    if (n < 0 || (n + 511) / 512 > 0x7FFFFFFF) return EXL3C4_E_SHAPE;
    if (n == 0) return 0;
    hipLaunchKernelGGL(k_narrow, dim3((unsigned)((n + 511) / 512)), dim3(256), 0, (hipStream_t)stream, in, out_bf16,
                       out_f16, n);
    return launched();
}
