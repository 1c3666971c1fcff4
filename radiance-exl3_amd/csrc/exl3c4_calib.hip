// exl3c4_calib.hip -- the box's own ceilings, measured by this library's own kernels (libexl3c4_calib.so): the HBM
// read rate of a plain stream, the read rate of a list of extents (a decode step's live experts' planes, read the way
// the decode kernels read them), the VALU issue rate of the trellis decode's instructions, and the f16 MFMA rate of
// v_mfma_f32_16x16x32_f16. A measurement tool beside the product, as the reference keeps its own
// (tools/calib/stream.hip:1-15, tools/calib/peak.hip:1-16, tests/gpu/oprate.hip:1-10); nothing in libexl3c4.so
// calls it. Each entry times its kernel with HIP events on the caller's stream and returns the best of `reps`
// launches in milliseconds (negative: a HIP error).
#include <hip/hip_runtime.h>

#include <stdint.h>

namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

// A plain stream read: each thread reads 4 independent 16-byte words a round (all in flight before any use), the
// rounds striding the whole grid, and folds them by XOR; one word a workgroup goes out so nothing is dropped.
__global__ __launch_bounds__(256) void k_read(const u32x4_t* __restrict__ p, int64_t n16, uint32_t* out) {
    const int64_t stride = (int64_t)gridDim.x * 256;
    uint32_t acc = 0;
    int64_t j = (int64_t)blockIdx.x * 256 + threadIdx.x;
    for (; j + 3 * stride < n16; j += 4 * stride) {
        const u32x4_t a = p[j], b = p[j + stride], c = p[j + 2 * stride], d = p[j + 3 * stride];
        const u32x4_t x = a ^ b ^ c ^ d;
        acc ^= x.x ^ x.y ^ x.z ^ x.w;
    }
    for (; j < n16; j += stride) {
        const u32x4_t a = p[j];
        acc ^= a.x ^ a.y ^ a.z ^ a.w;
    }
    __shared__ uint32_t s[4];
    for (int d = 32; d >= 1; d >>= 1) acc ^= __shfl_xor(acc, d);
    if ((threadIdx.x & 63) == 0) s[threadIdx.x >> 6] = acc;
    __syncthreads();
    if (threadIdx.x == 0) out[blockIdx.x] = s[0] ^ s[1] ^ s[2] ^ s[3];
}

// A list of extents read as the decode kernels read a weight: each wave one run of `run` bytes (64 lanes x 16 bytes a
// step, the steps in order, two steps in flight), the runs of all extents dealt to the waves in order. ext[2 e] is the
// extent's address, ext[2 e + 1] its bytes (a multiple of `run`); first[e] the index of its first run.
__global__ __launch_bounds__(256) void k_read_runs(const uint64_t* __restrict__ ext, const int64_t* __restrict__ first,
                                                   int n_ext, int64_t n_runs, int run, uint32_t* out) {
    const int lane = threadIdx.x & 63;
    const int64_t w = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    uint32_t acc = 0;
    if (w < n_runs) {
        int lo = 0, hi = n_ext - 1;                              // the extent holding run w
        while (lo < hi) {
            const int mid = (lo + hi + 1) / 2;
            if (first[mid] <= w) lo = mid;
            else hi = mid - 1;
        }
        const char* base = (const char*)ext[2 * lo] + (w - first[lo]) * run;
        const int steps = run / 1024;
        u32x4_t a = *(const u32x4_t*)(base + lane * 16);
        u32x4_t b = steps > 1 ? *(const u32x4_t*)(base + 1024 + lane * 16) : a;
        for (int s = 2; s < steps + 2; ++s) {
            const u32x4_t x = a;
            a = b;
            if (s < steps) b = *(const u32x4_t*)(base + (int64_t)s * 1024 + lane * 16);
            acc ^= x.x ^ x.y ^ x.z ^ x.w;
        }
    }
    for (int d = 32; d >= 1; d >>= 1) acc ^= __shfl_xor(acc, d);
    if (lane == 0 && acc == 0x9E3779B9u) out[0] = acc;             // almost never: keeps the reads live
}

// The decode's VALU instructions in 8 independent chains a wave (the issue rate, not the latency): each round is the
// mul1 pair sequence (2 v_pk_mul_lo_u16, 2 v_mad_u32_u16, v_sad_u8, v_sad_hi_u8, v_pk_fma_f16) on 8 register sets,
// 56 VALU instructions.
__global__ __launch_bounds__(256) void k_valu(int rounds, uint32_t seed, uint32_t* out) {
    uint32_t r[8], y[8];
    const uint32_t kh = 0x83DC0000u, cl = 0xD12Du, c64 = 0x64006400u, kinv = 0x1EEE1EEEu, kb = 0xC931C931u;
#pragma unroll
    for (int q = 0; q < 8; ++q) r[q] = seed ^ (threadIdx.x * 0x9E3779B9u) ^ (q * 0x85EBCA6Bu);
    for (int it = 0; it < rounds; ++it) {
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            uint32_t ya, yb;
            asm volatile(
                "v_pk_mul_lo_u16 %[ya], %[r], %[kh] op_sel:[0,0] op_sel_hi:[0,1]\n\t"
                "v_pk_mul_lo_u16 %[yb], %[r], %[kh] op_sel:[1,0] op_sel_hi:[1,1]\n\t"
                "v_mad_u32_u16 %[ya], %[r], %[cl], %[ya]\n\t"
                "v_mad_u32_u16 %[yb], %[r], %[cl], %[yb] op_sel:[1,0,0,0]\n\t"
                "v_sad_u8 %[ya], %[ya], 0, %[c64]\n\t"
                "v_sad_hi_u8 %[ya], %[yb], 0, %[ya]\n\t"
                "v_pk_fma_f16 %[r], %[ya], %[kinv], %[kb]"
                : [ya] "=&v"(ya), [yb] "=&v"(yb), [r] "+v"(r[q])
                : [kh] "s"(kh), [cl] "s"(cl), [c64] "s"(c64), [kinv] "s"(kinv), [kb] "v"(kb));
            y[q] = ya;
        }
    }
    uint32_t acc = 0;
#pragma unroll
    for (int q = 0; q < 8; ++q) acc ^= r[q] ^ y[q];
    if (acc == 0x9E3779B9u) out[0] = acc;
}

// v_mfma_f32_16x16x32_f16 in 8 independent accumulator chains a wave: 16 x 16 x 32 x 2 flops each.
__global__ __launch_bounds__(256) void k_mfma(int rounds, uint32_t* out) {
    float4_t acc[8];
    const half8_t a = { (_Float16)0.001f, (_Float16)0.002f, (_Float16)0.003f, (_Float16)0.004f,
                        (_Float16)0.005f, (_Float16)0.006f, (_Float16)0.007f, (_Float16)0.008f };
    const half8_t b = a * (_Float16)(threadIdx.x & 3);
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = float4_t{ 0.f, 0.f, 0.f, 0.f };
    for (int it = 0; it < rounds; ++it) {
#pragma unroll
        for (int q = 0; q < 8; ++q) acc[q] = __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, acc[q], 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int q = 0; q < 8; ++q) s += acc[q].x + acc[q].y + acc[q].z + acc[q].w;
    if (s == 12345.678f) out[0] = 1;
}

template <typename F> float best_ms(hipStream_t st, int reps, F launch) {
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return -1.f;
    launch();                                                     // untimed first launch
    float best = -1.f;
    for (int r = 0; r < reps; ++r) {
        (void)hipEventRecord(e0, st);
        launch();
        (void)hipEventRecord(e1, st);
        if (hipEventSynchronize(e1) != hipSuccess) { best = -1.f; break; }
        float ms = 0.f;
        (void)hipEventElapsedTime(&ms, e0, e1);
        if (best < 0.f || ms < best) best = ms;
    }
    (void)hipEventDestroy(e0);
    (void)hipEventDestroy(e1);
    return hipGetLastError() == hipSuccess ? best : -1.f;
}

}  // namespace

extern "C" {

// Reads `bytes` (a multiple of 16) at `p` with `blocks` workgroups of 256 threads; `scratch` holds a word a workgroup.
float exl3c4_calib_read(const void* p, int64_t bytes, int32_t blocks, void* scratch, int32_t reps, void* stream) {
    if (!p || bytes <= 0 || bytes % 16 || blocks <= 0 || !scratch) return -2.f;
    const hipStream_t st = (hipStream_t)stream;
    return best_ms(st, reps, [&] {
        hipLaunchKernelGGL(k_read, dim3((unsigned)blocks), dim3(256), 0, st, (const u32x4_t*)p, bytes / 16,
                           (uint32_t*)scratch);
    });
}

// Reads n_ext extents (device arrays: ext = {address, bytes} pairs, first = each extent's first run index, n_runs runs
// of `run` bytes in all, `run` a multiple of 1024) as the decode kernels read a weight, a wave a run.
float exl3c4_calib_read_runs(const void* ext, const void* first, int32_t n_ext, int64_t n_runs, int32_t run,
                             void* scratch, int32_t reps, void* stream) {
    if (!ext || !first || n_ext <= 0 || n_runs <= 0 || run <= 0 || run % 1024 || !scratch) return -2.f;
    const hipStream_t st = (hipStream_t)stream;
    return best_ms(st, reps, [&] {
        hipLaunchKernelGGL(k_read_runs, dim3((unsigned)((n_runs + 3) / 4)), dim3(256), 0, st, (const uint64_t*)ext,
                           (const int64_t*)first, n_ext, n_runs, run, (uint32_t*)scratch);
    });
}

// The decode's VALU mix: `blocks` workgroups of 4 waves, `rounds` rounds of 56 VALU instructions a wave.
float exl3c4_calib_valu(int32_t blocks, int32_t rounds, void* scratch, int32_t reps, void* stream) {
    if (blocks <= 0 || rounds <= 0 || !scratch) return -2.f;
    const hipStream_t st = (hipStream_t)stream;
    return best_ms(st, reps, [&] {
        hipLaunchKernelGGL(k_valu, dim3((unsigned)blocks), dim3(256), 0, st, rounds, 0x1234567u, (uint32_t*)scratch);
    });
}

// v_mfma_f32_16x16x32_f16: `blocks` workgroups of 4 waves, `rounds` rounds of 8 MFMAs a wave.
float exl3c4_calib_mfma(int32_t blocks, int32_t rounds, void* scratch, int32_t reps, void* stream) {
    if (blocks <= 0 || rounds <= 0 || !scratch) return -2.f;
    const hipStream_t st = (hipStream_t)stream;
    return best_ms(st, reps, [&] {
        hipLaunchKernelGGL(k_mfma, dim3((unsigned)blocks), dim3(256), 0, st, rounds, (uint32_t*)scratch);
    });
}

}  // extern "C"
