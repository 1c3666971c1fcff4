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

// f32 -> f16 bits, round to nearest even; the register fence keeps the conversion a conversion (not folded into the
// instruction that produced v).
__device__ __forceinline__ uint16_t to_f16(float v) {
    asm volatile("" : "+v"(v));
    return __builtin_bit_cast(uint16_t, (_Float16)v);
}

// The router's ranking as one unsigned 64-bit key a (logit, id): a larger key ranks first. The high word orders the
// logits (the sign-magnitude bits turned into an unsigned order; -0 taken as +0; a NaN below every number), the low
// word the ids (a lower id ranks first among equal logits).
__device__ __forceinline__ uint64_t rank_key(float l, int e) {
    uint32_t k = 0u;                                           // NaN
    if (l == l) {
        const uint32_t u = __float_as_uint(l == 0.f ? 0.f : l);
        k = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
    }
    return ((uint64_t)k << 32) | (uint64_t)(0xFFFFFFFFu - (uint32_t)e);
}
__device__ __forceinline__ float key_logit(uint64_t key) {
    const uint32_t k = (uint32_t)(key >> 32);
    return __uint_as_float((k & 0x80000000u) ? (k & 0x7FFFFFFFu) : ~k);
}

// The router for one token, by one wave: m = max logit; s = the sum of expf(l - m) (each lane over its ids e = lane +
// 64 j in ascending j, then a butterfly over the lanes); the top_k rank keys; p = expf(l - m) / s, renormalised by the
// sum of the top_k p (in rank order) when asked. The token's logits sit in registers (RPL a lane, ids e = lane + 64 j),
// all loaded at once. Lane r < top_k ends holding the r-th ranked id and its weight. cand: 64 keys of LDS.
struct Pick { int id; float w; };
__device__ __forceinline__ uint64_t shfl_xor64(uint64_t v, int d) {
    return ((uint64_t)(uint32_t)__shfl_xor((int)(v >> 32), d) << 32) | (uint64_t)(uint32_t)__shfl_xor((int)(uint32_t)v, d);
}
// The value of lane l ^ J, without the LDS pipe's bpermute: DPP moves for J = 1, 2 (quad_perm) and 8 (row_ror 8), a
// ds_swizzle (xor mode, within 32 lanes) for 4, gfx950's permlane swaps for 16 and 32 (each lane takes the half of
// the swapped pair that came from its partner). Every lane of the wave must be active.
template <int J> __device__ __forceinline__ uint32_t xor_lane(uint32_t v, int lane) {
    if constexpr (J == 1) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false);
    else if constexpr (J == 2) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false);
    else if constexpr (J == 4) return (uint32_t)__builtin_amdgcn_ds_swizzle((int)v, 0x101F);
    else if constexpr (J == 8) return (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x128, 0xF, 0xF, false);
    else if constexpr (J == 16) {
        const auto r = __builtin_amdgcn_permlane16_swap(v, v, false, false);
        return (lane & 16) ? r[0] : r[1];
    } else {
        const auto r = __builtin_amdgcn_permlane32_swap(v, v, false, false);
        return (lane & 32) ? r[0] : r[1];
    }
}
template <int J> __device__ __forceinline__ uint64_t xor_lane64(uint64_t v, int lane) {
    return ((uint64_t)xor_lane<J>((uint32_t)(v >> 32), lane) << 32) | (uint64_t)xor_lane<J>((uint32_t)v, lane);
}
template <int J> __device__ __forceinline__ float xor_lanef(float v, int lane) {
    return __uint_as_float(xor_lane<J>(__float_as_uint(v), lane));
}
__device__ __forceinline__ uint64_t readlane64(uint64_t v, int l) {
    return ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(v >> 32), l) << 32) |
           (uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)v, l);
}
__device__ __forceinline__ uint32_t xor_lane_rt(uint32_t v, int j, int lane) {   // j a power of two <= 32
    switch (j) {
    case 1: return xor_lane<1>(v, lane);
    case 2: return xor_lane<2>(v, lane);
    case 4: return xor_lane<4>(v, lane);
    case 8: return xor_lane<8>(v, lane);
    case 16: return xor_lane<16>(v, lane);
    default: return xor_lane<32>(v, lane);
    }
}

// A bitonic sort of one u32 a lane across the wave, descending: lane 0 ends with the largest.
__device__ __forceinline__ uint32_t sort_desc32(uint32_t v, int lane) {
#pragma unroll
    for (int k = 2; k <= 64; k <<= 1)
#pragma unroll
        for (int j = k >> 1; j > 0; j >>= 1) {
            const uint32_t o = xor_lane_rt(v, j, lane);          // j is a constant once unrolled
            const bool take_max = ((lane & j) == 0) == ((lane & k) == 0);
            v = take_max ? max(o, v) : min(o, v);
        }
    return v;
}

// The inclusive sum of v over lanes 0 .. lane, by DPP: shifts within each row of 16 lanes, then the rows' totals by
// row broadcasts (lane 15 into row 1 and 3, lane 31 into rows 2 and 3). Every lane of the wave must be active.
__device__ __forceinline__ int wave_scan_incl(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);   // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);   // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);   // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);   // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);   // row_bcast:15 into rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);   // row_bcast:31 into rows 2, 3
    return v;
}

template <int DT, int RPL>                                      // RPL logits a lane: n_expert <= 64 RPL
__device__ __forceinline__ Pick route_token(const void* logits, int64_t row, int32_t n_expert, int32_t top_k,
                                            int32_t renorm, int lane, uint64_t* cand) {
    float v[RPL];
    if (DT == EXL3C4_F32) {
        const float* p = (const float*)logits + row;
#pragma unroll
        for (int j = 0; j < RPL; ++j) v[j] = lane + 64 * j < n_expert ? p[lane + 64 * j] : -INFINITY;
    } else {
        const uint16_t* p = (const uint16_t*)logits + row;
        uint16_t b[RPL];
#pragma unroll
        for (int j = 0; j < RPL; ++j) b[j] = lane + 64 * j < n_expert ? p[lane + 64 * j] : (uint16_t)0xFC00u;
#pragma unroll
        for (int j = 0; j < RPL; ++j)
            v[j] = DT == EXL3C4_BF16 ? __uint_as_float((uint32_t)b[j] << 16) : (float)__builtin_bit_cast(_Float16, b[j]);
        if (DT == EXL3C4_BF16)
#pragma unroll
            for (int j = 0; j < RPL; ++j)
                if (lane + 64 * j >= n_expert) v[j] = -INFINITY;
    }
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < RPL; ++j) m = fmaxf(m, v[j]);              // a NaN never wins
    m = fmaxf(m, xor_lanef<32>(m, lane));
    m = fmaxf(m, xor_lanef<16>(m, lane));
    m = fmaxf(m, xor_lanef<8>(m, lane));
    m = fmaxf(m, xor_lanef<4>(m, lane));
    m = fmaxf(m, xor_lanef<2>(m, lane));
    m = fmaxf(m, xor_lanef<1>(m, lane));
    float s = 0.f;
    uint64_t key[RPL];
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
        const bool in = lane + 64 * j < n_expert;
        s = s + (in ? expf(v[j] - m) : 0.f);
        key[j] = in ? rank_key(v[j], lane + 64 * j) : 0ull;     // 0: below every real key
    }
    s = s + xor_lanef<32>(s, lane);                               // the butterfly, partners 32, 16, .., 1
    s = s + xor_lanef<16>(s, lane);
    s = s + xor_lanef<8>(s, lane);
    s = s + xor_lanef<4>(s, lane);
    s = s + xor_lanef<2>(s, lane);
    s = s + xor_lanef<1>(s, lane);

    // The top_k keys all have a logit word of at least thr, the top_k-th largest logit word of the lanes' own largest
    // keys (top_k lanes hold a key that large; the logit word orders the keys, so a 32-bit sort finds it). Those
    // candidates -- at most 64 on this path -- are gathered one a lane and ranked; lane r then holds the r-th ranked
    // key. More than 64 (many equal logits in few lanes) take top_k rounds of a wave maximum.
    uint64_t lm = 0ull;
#pragma unroll
    for (int j = 0; j < RPL; ++j) lm = key[j] > lm ? key[j] : lm;
    const uint32_t thr = (uint32_t)__builtin_amdgcn_readlane((int)sort_desc32((uint32_t)(lm >> 32), lane), top_k - 1);
    int n = 0;
#pragma unroll
    for (int j = 0; j < RPL; ++j) {
        const bool c = key[j] != 0ull && (uint32_t)(key[j] >> 32) >= thr;
        const uint64_t bal = __ballot(c);
        const int at = n + (int)__builtin_amdgcn_mbcnt_hi((uint32_t)(bal >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)bal, 0));
        if (c && at < 64) cand[at] = key[j];
        n += __popcll(bal);
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    uint64_t mykey = 0ull;
    if (n <= 64) {
        // the candidates ranked (keys are distinct: the id is in the low bits), then placed by rank: lane r ends with
        // the r-th largest. n rounds of independent compares instead of a 64-lane sort's 21 dependent stages.
        const uint64_t ck = lane < n ? cand[lane] : 0ull;
        int rank = 0;
        for (int c = 0; c < n; ++c) rank += readlane64(ck, c) > ck ? 1 : 0;
        if (lane < n) cand[rank] = ck;                            // this wave's row alone: its LDS ops run in order
        asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
        mykey = lane < n ? cand[lane] : 0ull;
    } else {
        uint64_t prev = ~0ull;
        for (int r = 0; r < top_k; ++r) {
            uint64_t best = 0ull;
#pragma unroll
            for (int j = 0; j < RPL; ++j) best = (key[j] < prev && key[j] > best) ? key[j] : best;
#pragma unroll
            for (int d = 32; d >= 1; d >>= 1) {
                const uint64_t o = shfl_xor64(best, d);
                best = o > best ? o : best;
            }
            prev = best;
            if (lane == r) mykey = best;
        }
    }
    const float p = lane < top_k ? expf(key_logit(mykey) - m) / s : 0.f;
    float psum = 0.f;
    for (int r = 0; r < top_k; ++r) psum = psum + __builtin_bit_cast(float, __builtin_amdgcn_readlane(__float_as_int(p), r));   // rank order
    return Pick{ (int)(0xFFFFFFFFu - (uint32_t)mykey), renorm ? p / psum : p };
}

// The router, one wave a token (n_expert <= 1024).
template <int DT, int RPL>
__global__ __launch_bounds__(256) void k_router(const void* logits, int64_t n_tok, int32_t n_expert, int64_t pitch,
                                                int32_t top_k, int32_t renorm, int32_t* ids, float* w) {
    const int lane = threadIdx.x & 63;
    const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    __shared__ uint64_t cand[4][64];
    if (t >= n_tok) return;
    const Pick p = route_token<DT, RPL>(logits, t * pitch, n_expert, top_k, renorm, lane, cand[threadIdx.x >> 6]);
    if (lane < top_k) {
        ids[t * top_k + lane] = p.id;
        w[t * top_k + lane] = p.w;
    }
}

// moe_scatter by the first SC_WAVES waves of a workgroup; wave v owns the contiguous pairs [v * seg, (v + 1) * seg).
// Pass A counts, per wave, each expert's pairs (a lane's rank among the lanes of its 64-pair chunk with the same
// expert comes from a readlane sweep, and the last such lane adds the chunk's count); then expert_offset is the
// exclusive scan of the totals (each thread a run of experts, a scan across the lanes, then across the waves) and
// each wave's count becomes its first row for that expert; pass B places the pairs in order. `ids` may be in LDS.
// LDS: cnt[SC_WAVES][n_expert] i32 and SC_WAVES wave sums. Every thread of the workgroup calls it (barriers).
constexpr int SC_WAVES = 8;
__device__ __forceinline__ void rank_in_chunk(int e, int lane, int n, int& rank, bool& last) {
    rank = 0;
    last = true;
    for (int q = 0; q < n; ++q) {                                // the chunk's n valid lanes

        const bool same = __builtin_amdgcn_readlane(e, q) == e;
        rank += (same && q < lane) ? 1 : 0;
        last = last && !(same && q > lane);
    }
}

__device__ __forceinline__ int expert_of(const int32_t* ids, int i, int hi, int64_t base, int n_expert) {
    if (i >= hi) return -1;
    const int64_t g = (int64_t)ids[i] - base;
    return (g >= 0 && g < n_expert) ? (int)g : -1;
}

__device__ void scatter_body(const int32_t* ids, int T, int64_t base, int n_expert, int32_t* sorted, int32_t* off,
                             int32_t* count, int32_t* row_of, int* cnt, int* wsum) {
    const int tid = threadIdx.x, lane = tid & 63, v = tid >> 6;
    const int nthr = SC_WAVES * 64;
    const bool act = v < SC_WAVES;
    const int seg = (T + SC_WAVES - 1) / SC_WAVES;
    const int lo = v * seg, hi = lo + seg < T ? lo + seg : T;
    for (int j = tid; j < SC_WAVES * n_expert; j += blockDim.x) cnt[j] = 0;
    __syncthreads();
    if (act)
        for (int c0 = lo; c0 < hi; c0 += 64) {                   // pass A
            const int e = expert_of(ids, c0 + lane, hi, base, n_expert);
            int rank;
            bool last;
            rank_in_chunk(e, lane, hi - c0 < 64 ? hi - c0 : 64, rank, last);
            if (e >= 0 && last) cnt[v * n_expert + e] += rank + 1;
        }
    __syncthreads();
    const int per = (n_expert + nthr - 1) / nthr;                 // thread tid: experts [tid * per, (tid + 1) * per)
    int mine = 0;
    if (act)
        for (int e = tid * per; e < (tid + 1) * per && e < n_expert; ++e)
            for (int u = 0; u < SC_WAVES; ++u) mine += cnt[u * n_expert + e];
    int incl = mine;                                              // inclusive scan across the wave's lanes
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
    }
    if (act && lane == 63) wsum[v] = incl;
    __syncthreads();
    int run = incl - mine;                                        // rows before this thread's first expert
    for (int u = 0; u < v && u < SC_WAVES; ++u) run += wsum[u];
    int live = 0;
    for (int u = 0; u < SC_WAVES; ++u) live += wsum[u];
    if (act)
        for (int e = tid * per; e < (tid + 1) * per && e < n_expert; ++e) {
            off[e] = run;
            int tot = 0;
            for (int u = 0; u < SC_WAVES; ++u) {                  // each wave's first row for expert e
                const int c = cnt[u * n_expert + e];
                cnt[u * n_expert + e] = run + tot;
                tot += c;
            }
            if (count) count[e] = tot;
            run += tot;
        }
    if (tid == 0) off[n_expert] = live;
    __syncthreads();
    if (act)
        for (int c0 = lo; c0 < hi; c0 += 64) {                   // pass B
            const int i = c0 + lane;
            const int e = expert_of(ids, i, hi, base, n_expert);
            int rank;
            bool last;
            rank_in_chunk(e, lane, hi - c0 < 64 ? hi - c0 : 64, rank, last);
            if (i < hi) {
                int pos = -1;
                if (e >= 0) {
                    pos = cnt[v * n_expert + e] + rank;
                    sorted[pos] = i;
                }
                if (row_of) row_of[i] = pos;
            }
            __builtin_amdgcn_wave_barrier();
            if (e >= 0 && last) cnt[v * n_expert + e] += rank + 1;
        }
    for (int i = live + tid; i < T; i += blockDim.x) sorted[i] = -1;
}

__global__ __launch_bounds__(512) void k_scatter(const int32_t* ids, int32_t T, int64_t base, int32_t n_expert,
                                                 int32_t* sorted, int32_t* off, int32_t* count, int32_t* row_of) {
    extern __shared__ int sc_lds[];
    scatter_body(ids, T, base, n_expert, sorted, off, count, row_of, sc_lds, sc_lds + SC_WAVES * n_expert);
}

// moe_scatter of the router's pairs (token t's top_k ids at t * top_k .., distinct experts, at most 32 tokens and
// blockDim.x pairs) for at most blockDim.x experts: each expert's set of tokens as a bit mask (LDS atomics), its count
// the mask's population; expert_offset the counts' exclusive scan (a DPP scan in each wave, then the waves' totals
// scanned the same way); pair (t, slot)'s row = offset of its expert + the number of earlier tokens holding that
// expert (the stable counting sort's row: a token holds an expert at most once, so the pairs of one expert are in
// token order). lds: n_expert + 1 + 16 ints, the first n_expert zeroed by the caller before a barrier.
__device__ __forceinline__ void scatter_small(const int32_t* ids_l, int T, int top_k, int n_expert, int32_t* sorted,
                                              int32_t* off, int32_t* count, int32_t* row_of, int* lds) {
    const int tid = threadIdx.x, lane = tid & 63, wv = tid >> 6;
    int* cnt = lds;                                               // [n_expert]: token masks, then exclusive offsets
    int* wsum = lds + n_expert + 1;                               // [16]: the waves' totals
    int e = -1, w = 0;
    const int t = tid < T ? tid / top_k : 0;
    if (tid < T) {
        const int f = ids_l[tid];
        e = (f >= 0 && f < n_expert) ? f : -1;
        if (e >= 0) atomicOr((unsigned*)&cnt[e], 1u << t);
    }
    __syncthreads();
    const int c = tid < n_expert ? __popc((unsigned)cnt[tid]) : 0;
    if (e >= 0) w = __popc((unsigned)cnt[e] & ((1u << t) - 1u));  // read before any offset overwrites a mask
    const int incl = wave_scan_incl(c);                           // inclusive scan across the wave
    if (lane == 63) wsum[wv] = incl;
    __syncthreads();
    const int nw = (int)(blockDim.x >> 6);                        // the waves' totals, lane u holding wave u's,
    const int pre = wave_scan_incl(lane < nw ? wsum[lane] : 0);   // scanned across lanes (at most 16 waves)
    const int base = wv ? __builtin_amdgcn_readlane(pre, wv - 1) : 0, live = __builtin_amdgcn_readlane(pre, nw - 1);
    if (tid < n_expert) {
        const int ex = base + incl - c;
        off[tid] = ex;
        if (count) count[tid] = c;
        cnt[tid] = ex;                                            // every read of the masks lies before the barrier
    }
    if (tid == 0) off[n_expert] = live;
    __syncthreads();
    if (tid < T) {
        const int rank = e >= 0 ? cnt[e] + w : -1;
        if (e >= 0) sorted[rank] = tid;
        if (row_of) row_of[tid] = rank;
    }
    for (int i = live + tid; i < T; i += blockDim.x) sorted[i] = -1;
}

// router_topk_scatter (the two fused, as the contract names them, include/exl3_abi.h:96-98) for at most 16 tokens, in
// one workgroup of 16 waves: wave t routes token t, its ids go to LDS as well, then the scatter reads them there.
template <int DT, int RPL>
__global__ __launch_bounds__(1024) void k_route_scatter(const void* logits, int32_t n_tok, int32_t n_expert,
                                                        int64_t pitch, int32_t top_k, int32_t renorm, int32_t* ids,
                                                        float* w, int32_t* sorted, int32_t* off, int32_t* count,
                                                        int32_t* row_of) {
    extern __shared__ __attribute__((aligned(16))) int rs_lds[];   // ids first: 16-byte reads
    __shared__ uint64_t cand[16][64];
    int* ids_l = rs_lds;                                          // [16 * 64]
    int* cnt = rs_lds + 16 * 64;
    const int lane = threadIdx.x & 63, t = threadIdx.x >> 6;
    const bool small = n_tok <= 32 && n_tok * top_k <= (int)blockDim.x && n_expert <= (int)blockDim.x;
    if (small)                                                    // the histogram's counts, zeroed while routing
        for (int i = threadIdx.x; i < n_expert; i += blockDim.x) cnt[i] = 0;
    if (t < n_tok) {
        const Pick p = route_token<DT, RPL>(logits, (int64_t)t * pitch, n_expert, top_k, renorm, lane, cand[t]);
        if (lane < top_k) {
            ids[t * top_k + lane] = p.id;
            w[t * top_k + lane] = p.w;
            ids_l[t * top_k + lane] = p.id;
        }
    }
    __syncthreads();
    if (small) scatter_small(ids_l, n_tok * top_k, top_k, n_expert, sorted, off, count, row_of, cnt);
    else scatter_body(ids_l, n_tok * top_k, 0, n_expert, sorted, off, count, row_of, cnt, cnt + SC_WAVES * n_expert);
}

// moe_gather: one thread a run of 8 columns of one token; the slots in ascending order, one f32 product and one add
// each, then f16. The rows and weights of 8 slots are read together, then their rows' values.
__global__ __launch_bounds__(256) void k_gather(const void* y, int32_t y_dtype, int64_t y_pitch, const float* w,
                                                const int32_t* row_of, int64_t n_tok, int32_t top_k, int64_t cols,
                                                uint16_t* out, int64_t out_pitch) {
    const int64_t t = blockIdx.x;
    const int64_t c = ((int64_t)blockIdx.y * 256 + threadIdx.x) * 8;
    if (t >= n_tok || c >= cols) return;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.f;
    for (int s0 = 0; s0 < top_k; s0 += 8) {                      // (every load unconditional: no branches)
        int32_t r[8];
        float ws[8];
        uint4 q[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const int sl = s0 + u < top_k ? s0 + u : top_k - 1;
            r[u] = row_of[t * top_k + sl];
            ws[u] = w[t * top_k + sl];
            if (s0 + u >= top_k) r[u] = -1;
        }
#pragma unroll
        for (int u = 0; u < 8; ++u)
            q[u] = *(const uint4*)((const uint16_t*)y + (int64_t)(r[u] < 0 ? 0 : r[u]) * y_pitch + c);
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            const uint32_t h[4] = { q[u].x, q[u].y, q[u].z, q[u].w };
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const uint16_t b = (uint16_t)(h[j >> 1] >> (16 * (j & 1)));
                const float v = y_dtype == EXL3C4_BF16 ? __uint_as_float((uint32_t)b << 16)
                                                       : (float)__builtin_bit_cast(_Float16, b);
                const float prod = ws[u] * v;
                const float sum = acc[j] + prod;
                acc[j] = r[u] < 0 ? acc[j] : sum;                     // a pair without a row adds nothing
            }
        }
    }
    uint32_t o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = (uint32_t)to_f16(acc[2 * j]) | ((uint32_t)to_f16(acc[2 * j + 1]) << 16);
    *(uint4*)(out + t * out_pitch + c) = uint4{ o[0], o[1], o[2], o[3] };
}

int launched() { return hipGetLastError() == hipSuccess ? 0 : EXL3C4_E_DEVICE; }

template <int DT, int RPL>
void launch_router(const void* logits, int64_t n_tok, int32_t n_expert, int64_t pitch, int32_t top_k, int32_t renorm,
                   int32_t* ids, float* w, hipStream_t st) {
    hipLaunchKernelGGL((k_router<DT, RPL>), dim3((unsigned)((n_tok + 3) / 4)), dim3(256), 0, st, logits, n_tok,
                       n_expert, pitch, top_k, renorm, ids, w);
}
template <int DT>
void launch_router_dt(const void* logits, int64_t n_tok, int32_t n_expert, int64_t pitch, int32_t top_k,
                      int32_t renorm, int32_t* ids, float* w, hipStream_t st) {
    if (n_expert <= 64) launch_router<DT, 1>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, st);
    else if (n_expert <= 128) launch_router<DT, 2>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, st);
    else if (n_expert <= 256) launch_router<DT, 4>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, st);
    else if (n_expert <= 512) launch_router<DT, 8>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, st);
    else launch_router<DT, 16>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, st);
}

template <int DT, int RPL>
void launch_rs(const void* logits, int32_t n_tok, int32_t n_expert, int64_t pitch, int32_t top_k, int32_t renorm,
               int32_t* ids, float* w, int32_t* sorted, int32_t* off, int32_t* count, int32_t* row_of, uint32_t lds,
               hipStream_t st) {
    hipLaunchKernelGGL((k_route_scatter<DT, RPL>), dim3(1), dim3(1024), lds, st, logits, n_tok, n_expert, pitch, top_k,
                       renorm, ids, w, sorted, off, count, row_of);
}
template <int DT>
void launch_rs_dt(const void* logits, int32_t n_tok, int32_t n_expert, int64_t pitch, int32_t top_k, int32_t renorm,
                  int32_t* ids, float* w, int32_t* sorted, int32_t* off, int32_t* count, int32_t* row_of,
                  uint32_t lds, hipStream_t st) {
    if (n_expert <= 64) launch_rs<DT, 1>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, sorted, off, count, row_of, lds, st);
    else if (n_expert <= 128) launch_rs<DT, 2>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, sorted, off, count, row_of, lds, st);
    else if (n_expert <= 256) launch_rs<DT, 4>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, sorted, off, count, row_of, lds, st);
    else if (n_expert <= 512) launch_rs<DT, 8>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, sorted, off, count, row_of, lds, st);
    else launch_rs<DT, 16>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, sorted, off, count, row_of, lds, st);
}

}  // namespace

extern "C" int exl3c4_dev_router(const void* logits, int32_t dtype, int64_t n_tok, int32_t n_expert, int64_t pitch,
                                 int32_t top_k, int32_t renorm, int32_t* ids, float* w, void* stream) {
    if (n_tok <= 0) return 0;
    const hipStream_t st = (hipStream_t)stream;
    if (dtype == EXL3C4_F32) launch_router_dt<EXL3C4_F32>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, st);
    else if (dtype == EXL3C4_BF16) launch_router_dt<EXL3C4_BF16>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, st);
    else launch_router_dt<EXL3C4_F16>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, st);
    return launched();
}

extern "C" int exl3c4_dev_scatter(const int32_t* ids, int64_t T, int64_t base, int32_t n_expert, int32_t* sorted,
                                  int32_t* off, int32_t* count, int32_t* row_of, void* stream) {
    const uint32_t lds = (uint32_t)((SC_WAVES * n_expert + SC_WAVES) * 4);
    hipLaunchKernelGGL(k_scatter, dim3(1), dim3(SC_WAVES * 64), lds, (hipStream_t)stream, ids, (int32_t)T, base,
                       n_expert, sorted, off, count, row_of);
    return launched();
}

extern "C" int exl3c4_dev_route_scatter(const void* logits, int32_t dtype, int32_t n_tok, int32_t n_expert,
                                        int64_t pitch, int32_t top_k, int32_t renorm, int32_t* ids, float* w,
                                        int32_t* sorted, int32_t* off, int32_t* count, int32_t* row_of,
                                        void* stream) {
    const int tail = SC_WAVES * n_expert + SC_WAVES > n_expert + 17 ? SC_WAVES * n_expert + SC_WAVES : n_expert + 17;
    const uint32_t lds = (uint32_t)((16 * 64 + tail) * 4);       // ids, then scatter_body's or scatter_small's
    const hipStream_t st = (hipStream_t)stream;
    if (dtype == EXL3C4_F32)
        launch_rs_dt<EXL3C4_F32>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, sorted, off, count, row_of, lds, st);
    else if (dtype == EXL3C4_BF16)
        launch_rs_dt<EXL3C4_BF16>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, sorted, off, count, row_of, lds, st);
    else
        launch_rs_dt<EXL3C4_F16>(logits, n_tok, n_expert, pitch, top_k, renorm, ids, w, sorted, off, count, row_of, lds, st);
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
