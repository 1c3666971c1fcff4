// exl3c4_route.hip -- the routing around the routed-expert ops, on gfx950 (wave64): the router (softmax over all
// logits, top_k, renormalisation), moe_scatter (a stable counting sort of the flat (token, slot) pairs by expert) and
// moe_gather (each token's slots weighted and summed in f32, ascending slot order, cast to f16). The contract is
// radiance's (include/exl3_abi.h:90-158; the scatter as tests/ref/exl3_numpy.py:223-242 states it); the reference
// device library leaves these to its engine.
#include <hip/hip_runtime.h>

#include <math.h>
#include <stdint.h>

#include "exl3c4_dev.h"

namespace {

__device__ __forceinline__ float load_logit(const void* p, int dtype, int64_t idx) {
    if (dtype == EXL3C4_F32) return ((const float*)p)[idx];
    const uint16_t b = ((const uint16_t*)p)[idx];
    if (dtype == EXL3C4_BF16) return __uint_as_float((uint32_t)b << 16);
    return (float)__builtin_bit_cast(_Float16, b);
}

// f32 -> f16 bits, round to nearest even; the register fence keeps the conversion a conversion (not folded into the
// instruction that produced v).
__device__ __forceinline__ uint16_t to_f16(float v) {
    asm volatile("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// (logit, id) ordering of the router: a is ranked before b when its logit is larger, or equal with the lower id.
// A NaN logit ranks after every number.
__device__ __forceinline__ bool ranks_before(float la, int ea, float lb, int eb) {
    const bool na = la != la, nb = lb != lb;
    if (na != nb) return nb;
    if (!na && la != lb) return la > lb;
    return ea < eb;
}

// The router, one wave a token: m = max logit; s = the sum of expf(l - m) (each lane over its ids e = lane (mod 64)
// in ascending order, then a butterfly over the lanes); then top_k rounds, each the best-ranked id ranked after the
// previous round's; p = expf(l - m) / s, renormalised by the sum of the top_k p (in rank order) when asked.
__global__ __launch_bounds__(256) void k_router(const void* logits, int32_t dtype, int64_t n_tok, int32_t n_expert,
                                                int64_t pitch, int32_t top_k, int32_t renorm, int32_t* ids,
                                                float* w) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (t >= n_tok) return;
    const int64_t row = t * pitch;
    float m = -INFINITY;
    for (int e = lane; e < n_expert; e += 64) {
        const float l = load_logit(logits, dtype, row + e);
        m = l > m ? l : m;                                      // NaN never wins
    }
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) {
        const float o = __shfl_xor(m, d);
        m = o > m ? o : m;
    }
    float s = 0.f;
    for (int e = lane; e < n_expert; e += 64) s = s + expf(load_logit(logits, dtype, row + e) - m);
#pragma unroll
    for (int d = 32; d >= 1; d >>= 1) s = s + __shfl_xor(s, d);

    float prev_l = INFINITY, psum = 0.f, pk = 0.f;
    int prev_e = -1;
    for (int j = 0; j < top_k; ++j) {
        float bl = -INFINITY;
        int be = 0x7FFFFFFF;
        bool have = false;
        for (int e = lane; e < n_expert; e += 64) {
            const float l = load_logit(logits, dtype, row + e);
            if (j > 0 && !ranks_before(prev_l, prev_e, l, e)) continue;     // ranked already
            if (!have || ranks_before(l, e, bl, be)) { bl = l; be = e; have = true; }
        }
#pragma unroll
        for (int d = 32; d >= 1; d >>= 1) {
            const float ol = __shfl_xor(bl, d);
            const int oe = __shfl_xor(be, d);
            if (oe != 0x7FFFFFFF && (be == 0x7FFFFFFF || ranks_before(ol, oe, bl, be))) { bl = ol; be = oe; }
        }
        prev_l = bl;
        prev_e = be;
        const float p = expf(bl - m) / s;
        psum = psum + p;
        if (lane == j) pk = p;
        if (lane == 0) ids[t * top_k + j] = be;
    }
    if (lane < top_k) w[t * top_k + lane] = renorm ? pk / psum : pk;
}

// moe_scatter in one workgroup of 8 waves; wave v owns the contiguous pairs [v * seg, (v + 1) * seg). Pass A counts,
// per wave, each expert's pairs (a lane's rank among the lanes of its 64-pair chunk with the same expert comes from a
// readlane sweep, and the last such lane adds the chunk's count); then expert_offset is the exclusive scan of the
// totals and each wave's count becomes its first row for that expert; pass B places the pairs in order. LDS:
// cnt[8][n_expert] i32, then the scan's 512 partial sums.
constexpr int SC_WAVES = 8;
__device__ __forceinline__ void rank_in_chunk(int e, int lane, int& rank, bool& last) {
    rank = 0;
    last = true;
    for (int q = 0; q < 64; ++q) {
        const int o = __builtin_amdgcn_readlane(e, q);
        if (o == e) {
            if (q < lane) ++rank;
            else if (q > lane) last = false;
        }
    }
}

__global__ __launch_bounds__(512) void k_scatter(const int32_t* ids, int64_t T, int64_t base, int32_t n_expert,
                                                 int32_t* sorted, int32_t* off, int32_t* count, int32_t* row_of) {
    extern __shared__ int sc_lds[];
    int* cnt = sc_lds;                                            // [SC_WAVES][n_expert]
    int* part = sc_lds + SC_WAVES * n_expert;                     // [512]
    const int tid = threadIdx.x, lane = tid & 63, v = tid >> 6;
    const int64_t seg = (T + SC_WAVES - 1) / SC_WAVES;
    const int64_t lo = v * seg, hi = lo + seg < T ? lo + seg : T;
    for (int j = tid; j < SC_WAVES * n_expert; j += 512) cnt[j] = 0;
    __syncthreads();
    for (int64_t c0 = lo; c0 < hi; c0 += 64) {                   // pass A
        const int64_t i = c0 + lane;
        int e = -1;
        if (i < hi) {
            const int64_t g = (int64_t)ids[i] - base;
            e = (g >= 0 && g < n_expert) ? (int)g : -1;
        }
        int rank;
        bool last;
        rank_in_chunk(e, lane, rank, last);
        if (e >= 0 && last) cnt[v * n_expert + e] += rank + 1;
    }
    __syncthreads();
    // the totals' exclusive scan: thread tid sums experts [tid * per, (tid + 1) * per)
    const int per = (n_expert + 511) / 512;
    int mine = 0;
    for (int e = tid * per; e < (tid + 1) * per && e < n_expert; ++e)
        for (int u = 0; u < SC_WAVES; ++u) mine += cnt[u * n_expert + e];
    part[tid] = mine;
    __syncthreads();
    for (int d = 1; d < 512; d <<= 1) {                           // inclusive scan of the partial sums
        const int o = tid >= d ? part[tid - d] : 0;
        __syncthreads();
        part[tid] += o;
        __syncthreads();
    }
    int run = part[tid] - mine;                                   // rows before this thread's first expert
    for (int e = tid * per; e < (tid + 1) * per && e < n_expert; ++e) {
        off[e] = run;
        int tot = 0;
        for (int u = 0; u < SC_WAVES; ++u) {                      // each wave's first row for expert e
            const int c = cnt[u * n_expert + e];
            cnt[u * n_expert + e] = run + tot;
            tot += c;
        }
        if (count) count[e] = tot;
        run += tot;
    }
    const int live = part[511];
    if (tid == 0) off[n_expert] = live;
    __syncthreads();
    for (int64_t c0 = lo; c0 < hi; c0 += 64) {                   // pass B
        const int64_t i = c0 + lane;
        int e = -1;
        if (i < hi) {
            const int64_t g = (int64_t)ids[i] - base;
            e = (g >= 0 && g < n_expert) ? (int)g : -1;
        }
        int rank;
        bool last;
        rank_in_chunk(e, lane, rank, last);
        if (i < hi) {
            int pos = -1;
            if (e >= 0) {
                pos = cnt[v * n_expert + e] + rank;
                sorted[pos] = (int32_t)i;
            }
            if (row_of) row_of[i] = pos;
        }
        __builtin_amdgcn_wave_barrier();
        if (e >= 0 && last) cnt[v * n_expert + e] += rank + 1;
    }
    for (int64_t i = live + tid; i < T; i += 512) sorted[i] = -1;
}

// moe_gather: one thread a run of 8 columns of one token; the slots in ascending order, one f32 product and one add
// each, then f16.
__global__ __launch_bounds__(256) void k_gather(const void* y, int32_t y_dtype, int64_t y_pitch, const float* w,
                                                const int32_t* row_of, int64_t n_tok, int32_t top_k, int64_t cols,
                                                uint16_t* out, int64_t out_pitch) {
    const int64_t t = blockIdx.x;
    const int64_t c = ((int64_t)blockIdx.y * 256 + threadIdx.x) * 8;
    if (t >= n_tok || c >= cols) return;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int s = 0; s < top_k; ++s) {
        const int32_t r = row_of[t * top_k + s];
        if (r < 0) continue;
        const float ws = w[t * top_k + s];
        const uint4 q = *(const uint4*)((const uint16_t*)y + (int64_t)r * y_pitch + c);
        const uint32_t h[4] = { q.x, q.y, q.z, q.w };
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const uint16_t b = (uint16_t)(h[j >> 1] >> (16 * (j & 1)));
            const float v = y_dtype == EXL3C4_BF16 ? __uint_as_float((uint32_t)b << 16)
                                                   : (float)__builtin_bit_cast(_Float16, b);
            const float prod = ws * v;
            acc[j] = acc[j] + prod;
        }
    }
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = (uint32_t)to_f16(acc[2 * j]) | ((uint32_t)to_f16(acc[2 * j + 1]) << 16);
    *(uint4*)(out + t * out_pitch + c) = uint4{ o[0], o[1], o[2], o[3] };
}

int launched() { return hipGetLastError() == hipSuccess ? 0 : EXL3C4_E_DEVICE; }

}  // namespace

extern "C" int exl3c4_dev_router(const void* logits, int32_t dtype, int64_t n_tok, int32_t n_expert, int64_t pitch,
                                 int32_t top_k, int32_t renorm, int32_t* ids, float* w, void* stream) {
    if (n_tok <= 0) return 0;
    hipLaunchKernelGGL(k_router, dim3((unsigned)((n_tok + 3) / 4)), dim3(256), 0, (hipStream_t)stream, logits, dtype,
                       n_tok, n_expert, pitch, top_k, renorm, ids, w);
    return launched();
}

extern "C" int exl3c4_dev_scatter(const int32_t* ids, int64_t T, int64_t base, int32_t n_expert, int32_t* sorted,
                                  int32_t* off, int32_t* count, int32_t* row_of, void* stream) {
    const uint32_t lds = (uint32_t)((SC_WAVES * n_expert + 512) * 4);
    hipLaunchKernelGGL(k_scatter, dim3(1), dim3(512), lds, (hipStream_t)stream, ids, T, base, n_expert, sorted, off,
                       count, row_of);
    return launched();
}

extern "C" int exl3c4_dev_gather(const void* y, int32_t y_dtype, int64_t y_pitch, const float* w,
                                 const int32_t* row_of, int64_t n_tok, int32_t top_k, int64_t cols, void* out,
                                 int64_t out_pitch, void* stream) {
    if (n_tok <= 0 || cols <= 0) return 0;
    hipLaunchKernelGGL(k_gather, dim3((unsigned)n_tok, (unsigned)((cols + 2047) / 2048)), dim3(256), 0,
                       (hipStream_t)stream, y, y_dtype, y_pitch, w, row_of, n_tok, top_k, cols, (uint16_t*)out,
                       out_pitch);
    return launched();
}
