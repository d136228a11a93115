// probe.hip -- hardware ceilings of gfx950 for the roofline of the RT4 path
// (librt4probe.so; measurement only, not part of the drop-in library).
//
// The reference measured its own target's ceilings with bench/bench_bw.cpp
// (HBM read probes) and bench/bench_isa2.cpp (dot-instruction issue rates) on
// gfx926; these are the gfx950 counterparts the benchmark reports next to the
// published MI355X peaks:
//   rt4p_hbm_read   streaming read of a buffer (dwordx4 loads, 8 in flight per lane)
//   rt4p_read_burst one-pass read of a buffer: each workgroup owns one slice and
//                   every lane issues all of its loads before using any (up to 16
//                   dwordx4 per lane), the access pattern of a single-launch weight
//                   stream; the ceiling a GEMV of that many bytes can reach
//   rt4p_copy       streaming copy of a buffer: a kernel of known traffic, used to
//                   calibrate rocprof's FETCH_SIZE / WRITE_SIZE counters
//   rt4p_mfma_i8    back-to-back v_mfma_i32_32x32x32_i8 / 16x16x64_i8 issue rate
//   rt4p_valu_fma   back-to-back v_fma_f32 issue rate (the GEMM's fold pipe)
#include <hip/hip_runtime.h>
#include <cstdint>

#include "rt4_probe.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(256) void hbm_read_k(const uint4* __restrict__ src, size_t n16,
                                                  uint32_t* __restrict__ sink) {
    constexpr int U = 8;
    const size_t stride = (size_t)gridDim.x * 256;
    uint32_t acc = 0;
    size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    for (; i + (U - 1) * stride < n16; i += U * stride) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; u++) v[u] = src[i + u * stride];
#pragma unroll
        for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    for (; i < n16; i += stride) {
        const uint4 v = src[i];
        acc ^= v.x ^ v.y ^ v.z ^ v.w;
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;  // practically never: keeps the loads live
}

// Workgroup b reads elements [b*chunk, (b+1)*chunk) of 16 bytes; lane t loads
// element b*chunk + u*blockDim + t for u < U, all before the first use.
typedef unsigned v4u __attribute__((ext_vector_type(4)));

template <int U, bool NT>
__global__ __launch_bounds__(1024) void read_burst_k(const v4u* __restrict__ src, size_t n16, size_t chunk,
                                                    uint32_t* __restrict__ sink) {
    const size_t base = (size_t)blockIdx.x * chunk;
    const size_t end = base + chunk < n16 ? base + chunk : n16;
    v4u v[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
        const size_t i = base + (size_t)u * blockDim.x + threadIdx.x;
        if (i < end)
            v[u] = NT ? __builtin_nontemporal_load(src + i) : src[i];
        else
            v[u] = v4u{0, 0, 0, 0};
    }
    uint32_t acc = 0;
#pragma unroll
    for (int u = 0; u < U; u++) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

template <bool NT>
hipError_t launch_burst(const v4u* src, size_t n16, uint32_t* sink, int blocks, int threads, int u,
                        hipStream_t st) {
    const size_t chunk = (n16 + blocks - 1) / blocks;
    switch (u) {
#define RT4P_B(U)                                                                                     \
    case U:                                                                                           \
        hipLaunchKernelGGL((read_burst_k<U, NT>), dim3(blocks), dim3(threads), 0, st, src, n16, chunk, \
                           sink);                                                                     \
        return hipGetLastError();
        RT4P_B(1) RT4P_B(2) RT4P_B(3) RT4P_B(4) RT4P_B(5) RT4P_B(6) RT4P_B(7) RT4P_B(8)
        RT4P_B(9) RT4P_B(10) RT4P_B(11) RT4P_B(12) RT4P_B(13) RT4P_B(14) RT4P_B(15) RT4P_B(16)
#undef RT4P_B
    }
    return hipErrorInvalidValue;
}

__global__ __launch_bounds__(256) void copy_k(uint4* __restrict__ dst, const uint4* __restrict__ src,
                                              size_t n16) {
    const size_t stride = (size_t)gridDim.x * 256;
    for (size_t i = (size_t)blockIdx.x * 256 + threadIdx.x; i < n16; i += stride) dst[i] = src[i];
}

// Each wave keeps 4 independent accumulator chains so the matrix pipe never
// waits on a dependency.
template <bool BIG>
__global__ __launch_bounds__(256) void mfma_i8_k(int32_t* __restrict__ sink, int iters, int seed) {
    const v4i a = {seed, (int)threadIdx.x, seed ^ 0x5A5A5A5A, 7};
    const v4i b = {(int)threadIdx.x * 3, seed, 11, seed >> 3};
    if (BIG) {
        v16i c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int it = 0; it < iters; it++) {
            c0 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, a, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, a, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_i32_32x32x32_i8(b, b, c3, 0, 0, 0);
        }
        int s = 0;
#pragma unroll
        for (int r = 0; r < 16; r++) s += c0[r] ^ c1[r] ^ c2[r] ^ c3[r];
        if (s == 0x13579BDF) sink[blockIdx.x] = s;
    } else {
        v4i c0 = {}, c1 = {}, c2 = {}, c3 = {};
        for (int it = 0; it < iters; it++) {
            c0 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c0, 0, 0, 0);
            c1 = __builtin_amdgcn_mfma_i32_16x16x64_i8(b, a, c1, 0, 0, 0);
            c2 = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, a, c2, 0, 0, 0);
            c3 = __builtin_amdgcn_mfma_i32_16x16x64_i8(b, b, c3, 0, 0, 0);
        }
        int s = 0;
#pragma unroll
        for (int r = 0; r < 4; r++) s += c0[r] ^ c1[r] ^ c2[r] ^ c3[r];
        if (s == 0x13579BDF) sink[blockIdx.x] = s;
    }
}

__global__ __launch_bounds__(256) void valu_fma_k(float* __restrict__ sink, int iters, float seed) {
    float x[8];
#pragma unroll
    for (int j = 0; j < 8; j++) x[j] = seed + (float)(threadIdx.x + j);
    const float m = 0.999f, a = 1e-7f;
    for (int it = 0; it < iters; it++)
#pragma unroll
        for (int j = 0; j < 8; j++) x[j] = fmaf(x[j], m, a);
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) s += x[j];
    if (s == 1234.5f) sink[blockIdx.x] = s;
}

hipError_t last() { return hipGetLastError(); }

}  // namespace

extern "C" {

int rt4p_hbm_read(const void* buf, size_t bytes, void* sink, int blocks, void* stream) {
    if (!buf || !sink || bytes % 16 || blocks < 1) return 1;
    hipLaunchKernelGGL(hbm_read_k, dim3(blocks), dim3(256), 0, (hipStream_t)stream,
                       (const uint4*)buf, bytes / 16, (uint32_t*)sink);
    return last() == hipSuccess ? 0 : 3;
}

int rt4p_read_burst(const void* buf, size_t bytes, void* sink, int blocks, int threads, int nontemporal,
                    void* stream) {
    if (!buf || !sink || bytes % 16 || blocks < 1 || threads < 64 || threads > 1024 || threads % 64) return 1;
    const size_t n16 = bytes / 16;
    const size_t chunk = (n16 + blocks - 1) / blocks;
    const size_t u = (chunk + threads - 1) / threads;
    if (u < 1 || u > 16) return 1;
    const hipError_t e = nontemporal ? launch_burst<true>((const v4u*)buf, n16, (uint32_t*)sink, blocks, threads,
                                                          (int)u, (hipStream_t)stream)
                                     : launch_burst<false>((const v4u*)buf, n16, (uint32_t*)sink, blocks, threads,
                                                           (int)u, (hipStream_t)stream);
    return e == hipSuccess ? 0 : 3;
}

int rt4p_copy(void* dst, const void* src, size_t bytes, int blocks, void* stream) {
    if (!dst || !src || bytes % 16 || blocks < 1) return 1;
    hipLaunchKernelGGL(copy_k, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (uint4*)dst,
                       (const uint4*)src, bytes / 16);
    return last() == hipSuccess ? 0 : 3;
}

int rt4p_mfma_i8(void* sink, int big, int iters, int blocks, void* stream) {
    if (!sink || iters < 1 || blocks < 1) return 1;
    if (big)
        hipLaunchKernelGGL(mfma_i8_k<true>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (int32_t*)sink,
                           iters, 12345);
    else
        hipLaunchKernelGGL(mfma_i8_k<false>, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (int32_t*)sink,
                           iters, 12345);
    return last() == hipSuccess ? 0 : 3;
}

int rt4p_valu_fma(void* sink, int iters, int blocks, void* stream) {
    if (!sink || iters < 1 || blocks < 1) return 1;
    hipLaunchKernelGGL(valu_fma_k, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (float*)sink, iters, 0.5f);
    return last() == hipSuccess ? 0 : 3;
}

}  // extern "C"
