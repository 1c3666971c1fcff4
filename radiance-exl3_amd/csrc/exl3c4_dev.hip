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
#include <utility>

#include "exl3c4_dev.h"

namespace {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half2_t __attribute__((ext_vector_type(2)));
typedef float    float4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4a_t __attribute__((ext_vector_type(4), aligned(4)));
typedef uint32_t u32x3a_t __attribute__((ext_vector_type(3), aligned(4)));
typedef uint32_t u32x2a_t __attribute__((ext_vector_type(2), aligned(4)));

constexpr float kHadScale = 0.08838834764831844055f;   // (float)(1/sqrt(128)), common/exl3_decode.c:173

// ------------------------------------------------------------------------------------------------ scalar helpers

__device__ __forceinline__ const void* tab_entry(const void* base, int64_t stride, int64_t j) {
    return stride ? (const void*)((const char*)base + j * stride) : ((const void* const*)base)[j];
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
// f32 -> f16, round to nearest even, of an f32 VALUE. The empty asm makes the operand a materialised f32 register:
// without it the backend folds a producing multiply into v_fma_mixlo_f16, which rounds the exact product to f16 once,
// where the reference rounds it to f32 first (a tie then lands on the other side, as measured on gfx950).
__device__ __forceinline__ uint16_t f2h(float f) {
    asm volatile("" : "+v"(f));
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}
__device__ __forceinline__ float bf2f(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }
// round to nearest even on the f32 bits (radiance's rad_f32_to_bf16); a nan stays a quiet nan
__device__ __forceinline__ uint16_t f2bf(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((u >> 16) | 0x40u);
    u += 0x7FFFu + ((u >> 16) & 1u);
    return (uint16_t)(u >> 16);
}

// The normalised Sylvester Hadamard over one 128-block held by a wave, lane l holding x[l] (v0) and x[l + 64] (v1):
// the butterfly stages h = 1 .. 64 in the reference's order, each (a + b) low and (a - b) high in f32, then one f32
// multiply by 1/sqrt(128) (common/exl3_decode.c:172-189) -- the same roundings, so the same bits.
__device__ __forceinline__ void had128_wave(float& v0, float& v1, int lane) {
#pragma unroll
    for (int h = 1; h < 64; h <<= 1) {
        const float p0 = __shfl_xor(v0, h), p1 = __shfl_xor(v1, h);
        const bool hi = (lane & h) != 0;
        v0 = hi ? p0 - v0 : v0 + p0;
        v1 = hi ? p1 - v1 : v1 + p1;
    }
    const float a = v0 + v1, b = v0 - v1;
    v0 = a * kHadScale;
    v1 = b * kHadScale;
}

// The expert owning sorted row i: e with off[e] <= i < off[e + 1], or -1 (include/exl3_abi.h:136-141). The offsets
// are device data nothing checked: a malformed table gives a wrong owner, never a read outside off[0 .. n_expert].
__device__ __forceinline__ int owner_of(const int32_t* off, int n_expert, int i) {
    if (i < off[0] || i >= off[n_expert]) return -1;
    int lo = 0, hi = n_expert;
    while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (off[mid] <= i) lo = mid;
        else hi = mid;
    }
    return lo;
}

__device__ __forceinline__ int dead_row(const Exl3c4Launch& a, int i, int* owner) {
    const int e = owner_of(a.off, a.n_expert, i);
    *owner = e;
    return e < 0 || a.sorted[i] < 0;
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

// h = x * 0x83DCD12D mod 2^32 for the state in half H of r: (x * 0x83DC mod 2^16) << 16 + x * 0xD12D.
template <int H> __device__ __forceinline__ uint32_t mul1_hash(uint32_t r, const Mul1Consts& k);
template <> __device__ __forceinline__ uint32_t mul1_hash<0>(uint32_t r, const Mul1Consts& k) {
    uint32_t y, h;
    asm("v_pk_mul_lo_u16 %0, %1, %2 op_sel:[0,0] op_sel_hi:[0,1]" : "=v"(y) : "v"(r), "s"(k.kh));
    asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[0,0,0,0]" : "=v"(h) : "v"(r), "s"(k.cl), "v"(y));
    return h;
}
template <> __device__ __forceinline__ uint32_t mul1_hash<1>(uint32_t r, const Mul1Consts& k) {
    uint32_t y, h;
    asm("v_pk_mul_lo_u16 %0, %1, %2 op_sel:[1,0] op_sel_hi:[1,1]" : "=v"(y) : "v"(r), "s"(k.kh));
    asm("v_mad_u32_u16 %0, %1, %2, %3 op_sel:[1,0,0,0]" : "=v"(h) : "v"(r), "s"(k.cl), "v"(y));
    return h;
}

// Two hashes -> two fp16 weights in one dword: low half from ha, high half from hb.
__device__ __forceinline__ uint32_t mul1_finish(uint32_t ha, uint32_t hb, const Mul1Consts& k) {
    uint32_t s = __builtin_amdgcn_sad_u8(ha, 0u, k.c6464);   // 0x6400 + bytesum(ha) | 0x6400 << 16
    s = __builtin_amdgcn_sad_hi_u8(hb, 0u, s);                // + bytesum(hb) << 16
    const half2_t v = __builtin_elementwise_fma(__builtin_bit_cast(half2_t, s), k.kinv, k.kbias);
    return __builtin_bit_cast(uint32_t, v);
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
        out = mul1_finish(mul1_hash<ha>(ra, k), mul1_hash<hb>(rb, k), k);
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

// One lane's segment -> its 32 weights as the four B operands (B[0..3] B_a, [4..7] B_b, [8..11] B_c, [12..15] B_d).
template <int BITS, int CB>
__device__ __forceinline__ void decode_segment(const uint32_t (&d)[BITS], uint32_t (&B)[16], const Mul1Consts& k) {
    uint32_t v[BITS + 1];
#pragma unroll
    for (int w = 0; w < BITS; ++w) v[w] = d[BITS - 1 - w];
    // the previous segment of the same tile: two lanes down, circularly within the 16-lane row (c = 2 s + t)
    v[BITS] = (uint32_t)__builtin_amdgcn_mov_dpp((int)d[BITS - 1], 0x122, 0xF, 0xF, false);
    decode_seg_impl<BITS, CB>(v, B, k, std::make_integer_sequence<int, 16>{});
}

// A lane's K words of one block: K u32 at p (4-byte aligned).
template <int BITS> __device__ __forceinline__ void load_words(const uint32_t* p, uint32_t (&d)[BITS]) {
    int w = 0;
#pragma unroll
    for (; w + 4 <= BITS; w += 4) {
        const u32x4a_t q = *(const u32x4a_t*)(p + w);
        d[w] = q.x; d[w + 1] = q.y; d[w + 2] = q.z; d[w + 3] = q.w;
    }
    if constexpr (BITS % 4 == 3) {
        const u32x3a_t q = *(const u32x3a_t*)(p + w);
        d[w] = q.x; d[w + 1] = q.y; d[w + 2] = q.z;
    } else if constexpr (BITS % 4 == 2) {
        const u32x2a_t q = *(const u32x2a_t*)(p + w);
        d[w] = q.x; d[w + 1] = q.y;
    } else if constexpr (BITS % 4 == 1) {
        d[w] = p[w];
    }
}

__device__ __forceinline__ half8_t as_half8(uint32_t a, uint32_t b, uint32_t c, uint32_t d) {
    return __builtin_bit_cast(half8_t, u32x4_t{ a, b, c, d });
}

// ------------------------------------------------------------------------------------------------ kernels

// The live chunks: every expert's run clamped to [0, T), cut into row blocks of at most 16, in expert order
// (the kernels clamp every run, kernels/exl3r4d/launch.c:14-15). One workgroup.
__global__ __launch_bounds__(256) void k_plan(const Exl3c4Launch a) {
    __shared__ int scan[256];
    __shared__ int carry_s;
    const int tid = threadIdx.x;
    if (tid == 0) carry_s = 0;
    __syncthreads();
    int4* ent = (int4*)(a.plan + 4);
    for (int base = 0; base < a.n_expert; base += 256) {
        const int e = base + tid;
        int lo = 0, hi = 0, n = 0;
        if (e < a.n_expert) {
            lo = min(max(a.off[e], 0), a.T);
            hi = min(max(a.off[e + 1], lo), a.T);
            n = (hi - lo + EXL3C4_CHUNK_ROWS - 1) / EXL3C4_CHUNK_ROWS;
        }
        scan[tid] = n;
        __syncthreads();
        for (int d = 1; d < 256; d <<= 1) {   // inclusive scan
            const int t = tid >= d ? scan[tid - d] : 0;
            __syncthreads();
            scan[tid] += t;
            __syncthreads();
        }
        const int carry = carry_s;
        const int first = carry + scan[tid] - n;
        for (int q = 0; q < n; ++q) {
            const int at = first + q;
            if (at < a.max_chunks) {
                const int r0 = lo + q * EXL3C4_CHUNK_ROWS;
                ent[at] = make_int4(e, r0, min(EXL3C4_CHUNK_ROWS, hi - r0), 0);
            }
        }
        __syncthreads();
        if (tid == 255) carry_s = carry + scan[255];
        __syncthreads();
    }
    if (tid == 0) a.plan[0] = min(carry_s, a.max_chunks);
}

// prep: one wave per (sorted row i, half m). Rows outside every run are not written (include/exl3_abi.h:273-278);
// a run's row whose sorted_tok is negative is written zero.
__global__ __launch_bounds__(256) void k_prep(const Exl3c4Launch a, int halves) {
    const int lane = threadIdx.x & 63;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t i = wid / halves;
    const int m = (int)(wid % halves);
    if (i >= a.T) return;
    const int e = owner_of(a.off, a.n_expert, (int)i);
    if (e < 0) return;
    const int c = e % a.n_class;
    const int64_t jx = e / a.n_class;
    const Exl3c4Class& K = a.cls[c];
    const int C = K.cols;
    const uint16_t* s = (const uint16_t*)(m ? tab_entry(K.suh1, K.suh1_stride, jx) : tab_entry(K.suh, K.suh_stride, jx));
    uint16_t* out = (uint16_t*)a.y + i * a.y_pitch + (int64_t)m * C;
    const int tok = a.sorted[i];
    if (tok < 0) {
        for (int k = lane; k < C; k += 64) out[k] = 0;
        return;
    }
    int64_t src = a.prep_mode == EXL3C4_PREP_DN ? i : tok / a.top_k;
    src = src < a.x_rows ? src : a.x_rows - 1;
    const uint16_t* x = (const uint16_t*)a.x + src * a.x_pitch;
    for (int b = 0; b < C; b += 128) {
        const uint16_t x0 = x[b + lane], x1 = x[b + 64 + lane];
        const float f0 = a.x_dtype == EXL3C4_BF16 ? bf2f(x0) : h2f(x0);
        const float f1 = a.x_dtype == EXL3C4_BF16 ? bf2f(x1) : h2f(x1);
        float v0 = h2f(f2h(f0 * h2f(s[b + lane])));
        float v1 = h2f(f2h(f1 * h2f(s[b + 64 + lane])));
        had128_wave(v0, v1, lane);
        out[b + lane] = f2h(v0);
        out[b + 64 + lane] = f2h(v1);
    }
}

// gemv: one wave per unit (chunk, 32-column strip, k split). Partial sums of the strip for the chunk's rows go to
// part[split][row][col]; the epilogue adds the splits in a fixed order, so the bits do not depend on scheduling.
template <int BITS, int CB>
__global__ __launch_bounds__(256) void k_gemv(const Exl3c4Launch a) {
    const int lane = threadIdx.x & 63;
    const int64_t unit = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int S = a.ksplit;
    const int split = (int)(unit % S);
    const int64_t t = unit / S;
    const int strip = (int)(t % a.max_strips);
    const int64_t chunk = t / a.max_strips;
    const int nch = min(a.plan[0], a.max_chunks);
    if (chunk >= nch) return;
    const int4 ent = ((const int4*)(a.plan + 4))[chunk];
    const int e = ent.x, row0 = ent.y, nrows = ent.z;
    const int c = e % a.n_class;
    const int64_t jx = e / a.n_class;
    const Exl3c4Class& K = a.cls[c];
    const int N = K.rows, KC = K.cols;
    if (strip * EXL3C4_STRIP >= N) return;
    const int ksteps = KC / EXL3C4_KSTEP;
    const int per = (ksteps + S - 1) / S;
    const int ks0 = split * per, ks1 = min(ksteps, ks0 + per);

    const uint32_t* rec = (const uint32_t*)tab_entry(K.codes, K.codes_stride, jx) + (int64_t)strip * ksteps * 64 * BITS;
    const int r = lane & 15, g = lane >> 4;
    const int i = row0 + r;
    bool valid = r < nrows;
    if (valid) valid = a.sorted[i] >= 0;
    const int acol = (a.gate_up && strip * EXL3C4_STRIP >= N / 2) ? KC : 0;
    const uint16_t* arow = (const uint16_t*)a.a + (int64_t)(valid ? i : 0) * a.a_pitch + acol + 16 * g;

    const Mul1Consts k = mul1_consts();
    float4_t acc0 = { 0.f, 0.f, 0.f, 0.f }, acc1 = { 0.f, 0.f, 0.f, 0.f };
    for (int ks = ks0; ks < ks1; ++ks) {
        uint32_t d[BITS];
        load_words<BITS>(rec + ((int64_t)ks * 64 + lane) * BITS, d);
        u32x4_t c0 = { 0, 0, 0, 0 }, c1 = { 0, 0, 0, 0 };
        if (valid) {
            c0 = *(const u32x4_t*)(arow + ks * EXL3C4_KSTEP);
            c1 = *(const u32x4_t*)(arow + ks * EXL3C4_KSTEP + 8);
        }
        uint32_t B[16];
        decode_segment<BITS, CB>(d, B, k);
        const half8_t Aa = as_half8(c0.x, c1.x, c0.y, c1.y), Ab = as_half8(c0.z, c1.z, c0.w, c1.w);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Aa, as_half8(B[0], B[1], B[2], B[3]), acc0, 0, 0, 0);
        acc0 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ab, as_half8(B[4], B[5], B[6], B[7]), acc0, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Aa, as_half8(B[8], B[9], B[10], B[11]), acc1, 0, 0, 0);
        acc1 = __builtin_amdgcn_mfma_f32_16x16x32_f16(Ab, as_half8(B[12], B[13], B[14], B[15]), acc1, 0, 0, 0);
    }
    // D lane l: column l % 16 (c' = 2 s + t -> weight row 32 nb + 16 t + s, + 8 for acc1), rows 4 (l / 16) + 0..3
    const int cc = lane & 15, rg = lane >> 4;
    const int n = strip * EXL3C4_STRIP + 16 * (cc & 1) + (cc >> 1);
    float* pp = a.part + (int64_t)split * a.part_split;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const int tok = rg * 4 + q;
        if (tok < nrows) {
            pp[(int64_t)(row0 + tok) * a.part_pitch + n] = acc0[q];
            pp[(int64_t)(row0 + tok) * a.part_pitch + n + 8] = acc1[q];
        }
    }
}

__device__ __forceinline__ float silu(float g) { return g * (1.0f / (1.0f + expf(-g))); }

__device__ __forceinline__ float sum_splits(const Exl3c4Launch& a, int64_t i, int col) {
    const float* p = a.part + i * a.part_pitch + col;
    float s = p[0];
    for (int q = 1; q < a.ksplit; ++q) s = s + p[(int64_t)q * a.part_split];
    return s;
}

// epilogue: one wave per (row i, 128-column block b of the output). Dead rows and a narrower class's tail are zero.
__global__ __launch_bounds__(256) void k_epilogue(const Exl3c4Launch a) {
    const int lane = threadIdx.x & 63;
    const int nblk = a.y_cols / 128;
    const int64_t wid = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    const int64_t i = wid / nblk;
    const int b = (int)(wid % nblk);
    if (i >= a.T) return;
    int e;
    const int dead = dead_row(a, (int)i, &e);
    uint16_t* out = (uint16_t*)a.y + i * a.y_pitch + b * 128;
    int width = 0, c = 0;
    int64_t jx = 0;
    if (!dead) {
        c = e % a.n_class;
        jx = e / a.n_class;
        width = a.gate_up ? a.cls[c].rows / 2 : a.cls[c].rows;
    }
    if (dead || b * 128 >= width) {
        out[lane] = 0;
        out[lane + 64] = 0;
        return;
    }
    const Exl3c4Class& K = a.cls[c];
    const uint16_t* svh = (const uint16_t*)tab_entry(K.svh, K.svh_stride, jx);
    const int n0 = b * 128 + lane, n1 = n0 + 64;
    if (a.gate_up) {
        float g0 = sum_splits(a, i, n0), g1 = sum_splits(a, i, n1);
        float u0 = sum_splits(a, i, width + n0), u1 = sum_splits(a, i, width + n1);
        had128_wave(g0, g1, lane);
        had128_wave(u0, u1, lane);
        g0 = g0 * h2f(svh[n0]);
        g1 = g1 * h2f(svh[n1]);
        u0 = u0 * h2f(svh[width + n0]);
        u1 = u1 * h2f(svh[width + n1]);
        const uint16_t h0 = f2h(silu(g0) * u0), h1 = f2h(silu(g1) * u1);
        if (!a.h_rot) {
            out[lane] = h0;
            out[lane + 64] = h1;
            return;
        }
        // h_rot = 1: down's first step, with down's suh of this expert (docs/OPS-exl3.md:120-123)
        const uint16_t* ds = (const uint16_t*)tab_entry(K.dn_suh, K.dn_suh_stride, jx);
        float v0 = h2f(f2h(h2f(h0) * h2f(ds[n0]))), v1 = h2f(f2h(h2f(h1) * h2f(ds[n1])));
        had128_wave(v0, v1, lane);
        out[lane] = f2h(v0);
        out[lane + 64] = f2h(v1);
    } else {
        float y0 = sum_splits(a, i, n0), y1 = sum_splits(a, i, n1);
        had128_wave(y0, y1, lane);
        out[lane] = f2bf(y0 * h2f(svh[n0]));
        out[lane + 64] = f2bf(y1 * h2f(svh[n1]));
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
    load_words<BITS>(rec + (blk * 64 + lane) * BITS, d);
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

typedef void (*GemvFn)(const Exl3c4Launch);
typedef void (*DequantFn)(const uint32_t*, int, int, uint16_t*, int64_t);

template <int BITS> GemvFn gemv_fn(int cb) {
    switch (cb) {
    case EXL3C4_CB_MUL1: return k_gemv<BITS, EXL3C4_CB_MUL1>;
    case EXL3C4_CB_MCG:  return k_gemv<BITS, EXL3C4_CB_MCG>;
    default:             return k_gemv<BITS, EXL3C4_CB_3INST>;
    }
}
template <int BITS> DequantFn dequant_fn(int cb) {
    switch (cb) {
    case EXL3C4_CB_MUL1: return k_dequant<BITS, EXL3C4_CB_MUL1>;
    case EXL3C4_CB_MCG:  return k_dequant<BITS, EXL3C4_CB_MCG>;
    default:             return k_dequant<BITS, EXL3C4_CB_3INST>;
    }
}

GemvFn pick_gemv(int bits, int cb) {
    switch (bits) {
    case 2: return gemv_fn<2>(cb);
    case 3: return gemv_fn<3>(cb);
    case 4: return gemv_fn<4>(cb);
    case 5: return gemv_fn<5>(cb);
    case 6: return gemv_fn<6>(cb);
    case 7: return gemv_fn<7>(cb);
    case 8: return gemv_fn<8>(cb);
    default: return nullptr;
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

}  // namespace

extern "C" int exl3c4_dev_plan(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    return go(k_plan, 1, (hipStream_t)stream, ev0, ev1, *a);
}

extern "C" int exl3c4_dev_prep(const Exl3c4Launch* a, int halves, void* stream, void* ev0, void* ev1) {
    const int64_t waves = (int64_t)a->T * halves;
    if (waves <= 0) return 0;
    return go(k_prep, blocks_for_waves(waves), (hipStream_t)stream, ev0, ev1, *a, halves);
}

extern "C" int exl3c4_dev_gemv(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    const GemvFn f = pick_gemv(a->bits, a->codebook);
    if (!f) return EXL3C4_E_DTYPE;
    const int64_t waves = (int64_t)a->max_chunks * a->max_strips * a->ksplit;
    if (waves <= 0) return 0;
    return go(f, blocks_for_waves(waves), (hipStream_t)stream, ev0, ev1, *a);
}

extern "C" int exl3c4_dev_epilogue(const Exl3c4Launch* a, void* stream, void* ev0, void* ev1) {
    const int64_t waves = (int64_t)a->T * (a->y_cols / 128);
    if (waves <= 0) return 0;
    return go(k_epilogue, blocks_for_waves(waves), (hipStream_t)stream, ev0, ev1, *a);
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
