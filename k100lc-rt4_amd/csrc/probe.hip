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
//   rt4p_gemv_loads the decode GEMV's own memory requests and nothing else: its
//                   grid (whole tiles plus K pieces of the leftover tiles), waves,
//                   per-chunk weight-scale dwords (or the hoisted ones), line-wise
//                   activation chunks and the non-temporal weight loads, in the
//                   2-group form (8 rows x 128 B per load), the row-transposed
//                   4-group form (4 rows x 256 B) or the one-row dot-product form
//                   (two rows per wave, 1 KB per load); the loaded words are only
//                   XOR-ed.  The gap between it and the GEMV is compute; the gap
//                   between it and rt4p_read_burst is the access pattern
//   rt4p_empty      an empty kernel: the per-launch cost of a graph node
//   rt4p_mfma_f8f6f4 back-to-back v_mfma_scale_f32_32x32x64_f8f6f4 with FP8, FP6 or
//                   FP4 operands (the matrix-core rate per format)
//   rt4p_mfma_f8_16x16 back-to-back v_mfma_f32_16x16x128_f8f6f4 (FP8, no block
//                   scale), the form the attention kernel issues, 8 chains per wave
//   rt4p_gemm_unit  the prefill GEMM's per-unit instruction skeleton without memory:
//                   per wave and 128-wide K group, four 32x32 row tiles of MFMAs with
//                   the previous row tile's fold interleaved, at the GEMM's occupancy
//                   (8 waves per CU); variant 0 the product's int8 form (16
//                   v_mfma_i32_32x32x32_i8, fold cvt + fma, the scale products as two
//                   two-block fp32 outer products per unit placed as in the GEMM),
//                   variant 1 an exact FP8-digit form (16
//                   v_mfma_scale_f32_32x32x64_f8f6f4 over two digit planes, fold one
//                   fma, a bias and a scale bf16 MFMA per row tile)
#include <hip/hip_runtime.h>
#include <cstdint>

#include "rt4_probe.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v16f __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef short v4h __attribute__((ext_vector_type(4)));

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

// ---- the decode GEMV's memory requests (rt4p_gemv_loads).  Mirrors gemv.hip's
// gemv_w4a8_k for one 16-row block per tile with line-wise activation loads
// (RB = 1, AL), the configuration of every configs[0..1] shape: tile / piece
// mapping, chunk distribution over the waves, and the three load streams with
// their address arithmetic; nothing is computed from the loaded words.
template <int M, int GPW, bool HS>
__global__ __launch_bounds__(1024) void gemv_loads_k(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                                                     const int8_t* __restrict__ xq, uint32_t* __restrict__ sink,
                                                     int N, int K, int full, int nrem, int S) {
    constexpr int NP = GPW / 2, ACH = M * GPW * 8, AIN = (ACH + 63) / 64;
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15, q = lane >> 4;
    const int NG = K >> 7, RS = K >> 1, NC = (NG + GPW - 1) / GPW;
    const int b = blockIdx.x, npieces = nrem * S;
    const bool piece = b < npieces;
    const int rem = piece ? b / S : 0, pc = piece ? b % S : 0;
    const int tile = piece ? full + rem : b - npieces;
    const int c_lo = piece ? pc * NC / S : 0, c_hi = piece ? (pc + 1) * NC / S : NC;
    const int n0 = tile * 16;
    const bool lo = j < 8;
    int r1 = n0 + (lo ? j : j - 8), r2 = n0 + (lo ? j + 8 : j);
    r1 = r1 < N ? r1 : N - 1;
    r2 = r2 < N ? r2 : N - 1;
    const unsigned char* p1 = reinterpret_cast<const unsigned char*>(wq) + (size_t)r1 * RS + (lo ? q : 4 + q) * 16;
    const unsigned char* p2 = reinterpret_cast<const unsigned char*>(wq) + (size_t)r2 * RS + (lo ? 4 + q : q) * 16;
    const int rj = n0 + j < N ? n0 + j : N - 1;
    uint32_t acc = 0;
    if (HS) {
#pragma unroll
        for (int i = 0; i < 2; i++) {
            int c = c_lo + w + (q + 4 * i) * W;
            c = c < c_hi ? c : c_lo;
            acc ^= *reinterpret_cast<const uint32_t*>(ws + (size_t)rj * NG + 2 * c);
        }
    }
    for (int c = c_lo + w; c < c_hi; c += W) {
        const int g0 = __builtin_amdgcn_readfirstlane(c * GPW);
        uint32_t sw = 0;
        if (!HS) {
#pragma unroll
            for (int d = 0; d < (GPW / 2 + 3) / 4; d++) {
                const int dw = q + 4 * d, g = g0 + 2 * dw;
                if (dw < GPW / 2 && g < NG) sw ^= *reinterpret_cast<const uint32_t*>(ws + (size_t)rj * NG + g);
            }
        }
        uint4 araw[AIN];
#pragma unroll
        for (int i = 0; i < AIN; i++) {
            int e = i * 64 + lane;
            e = e < ACH ? e : ACH - 1;
            const int row = e / (GPW * 8), grp = (e / 8) % GPW, cc = e % 8;
            int g = g0 + grp;
            g = g < NG ? g : NG - 1;
            araw[i] = *reinterpret_cast<const uint4*>(xq + (size_t)row * K + (size_t)g * 128 + cc * 16);
        }
        v4u a[NP], bb[NP];
#pragma unroll
        for (int p = 0; p < NP; p++) {
            int gp = g0 + 2 * p;
            if (gp >= NG) gp = NG >= 2 ? NG - 2 : 0;
            const int tail = (gp + 1 >= NG) ? 64 : 0;
            a[p] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p1 + (size_t)gp * 64 - (lo ? 0 : tail)));
            bb[p] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p2 + (size_t)gp * 64 - (lo ? tail : 0)));
        }
        acc ^= sw;
#pragma unroll
        for (int i = 0; i < AIN; i++) acc ^= araw[i].x ^ araw[i].y ^ araw[i].z ^ araw[i].w;
#pragma unroll
        for (int p = 0; p < NP; p++) acc ^= a[p].x ^ a[p].y ^ a[p].z ^ a[p].w ^ bb[p].x ^ bb[p].y ^ bb[p].z ^ bb[p].w;
    }
    if (acc == 0x9E3779B9u) sink[b] = acc;   // practically never: keeps the loads live
}

// The row-transposed GEMV's requests (gemv.hip gemv_w4a8_tl_k): 4 groups per
// chunk, one chunk per wave at a time, its scale dwords, activation lines and four
// non-temporal 4-row x 256 B weight loads with the kernel's lane-to-piece mapping.
template <int M>
__global__ __launch_bounds__(512) void gemv_loads_tl_k(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                                                       const int8_t* __restrict__ xq, uint32_t* __restrict__ sink,
                                                       int N, int K, int full, int nrem, int S) {
    constexpr int GPW = 4, ACH = M * GPW * 8, AIN = (ACH + 63) / 64;
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int j = lane & 15;
    const int NG = K >> 7, RS = K >> 1, NC = NG >> 2;
    const int b = blockIdx.x, npieces = nrem * S;
    const bool piece = b < npieces;
    const int rem = piece ? b / S : 0, pc = piece ? b % S : 0;
    const int tile = piece ? full + rem : b - npieces;
    const int c_lo = piece ? pc * NC / S : 0, c_hi = piece ? (pc + 1) * NC / S : NC;
    const int n0 = tile * 16;
    const unsigned char* pk[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int rho = 4 * k + (lane >> 4);
        int r = n0 + rho;
        r = r < N ? r : N - 1;
        pk[k] = reinterpret_cast<const unsigned char*>(wq) + (size_t)r * RS + (((lane & 15) ^ rho) * 16);
    }
    const uint16_t* wsr = ws + (size_t)(n0 + j < N ? n0 + j : N - 1) * NG;
    uint32_t acc = 0;
    for (int c = c_lo + w; c < c_hi; c += W) {
        const int g0 = __builtin_amdgcn_readfirstlane(c * GPW);
        const uint32_t s0 = *reinterpret_cast<const uint32_t*>(wsr + g0);
        const uint32_t s1 = *reinterpret_cast<const uint32_t*>(wsr + g0 + 2);
        v4u araw[AIN], wv[4];
#pragma unroll
        for (int t = 0; t < AIN; t++) {
            int e = t * 64 + lane;
            e = e < ACH ? e : ACH - 1;
            const int row = e / (GPW * 8), grp = (e / 8) % GPW, cc = e % 8;
            araw[t] = *reinterpret_cast<const v4u*>(xq + (size_t)row * K + (size_t)(g0 + grp) * 128 + cc * 16);
        }
#pragma unroll
        for (int k = 0; k < 4; k++) wv[k] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(pk[k] + (size_t)g0 * 64));
        acc ^= s0 ^ s1;
#pragma unroll
        for (int t = 0; t < AIN; t++) acc ^= araw[t].x ^ araw[t].y ^ araw[t].z ^ araw[t].w;
#pragma unroll
        for (int k = 0; k < 4; k++) acc ^= wv[k].x ^ wv[k].y ^ wv[k].z ^ wv[k].w;
    }
    if (acc == 0x9E3779B9u) sink[b] = acc;   // practically never: keeps the loads live
}

// The one-row dot-product GEMV's requests (gemv.hip gemv_w4a8_dot_k): two weight
// rows per wave read as consecutive 1 KB load instructions, each lane's 32 matching
// activation bytes, and the wave's scale dwords loaded once.
template <int NI>
__global__ __launch_bounds__(256) void gemv_loads_dot_k(const uint32_t* __restrict__ wq, const uint16_t* __restrict__ ws,
                                                        const int8_t* __restrict__ xq, const float* __restrict__ sa,
                                                        uint32_t* __restrict__ sink, int N, int K) {
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6)));
    const int NG = K >> 7, RS = K >> 1;
    const int n0 = wv * 2;
    if (n0 >= N) return;
    const int nrows = min(2, N - n0);
    const int span = nrows * RS;
    const unsigned char* wb = reinterpret_cast<const unsigned char*>(wq) + (size_t)n0 * RS;
    const int nsw = (nrows * NG + 1) >> 1;
    uint32_t acc = lane < nsw ? reinterpret_cast<const uint32_t*>(ws + (size_t)n0 * NG)[lane] : 0u;
    acc ^= lane < NG ? __float_as_uint(sa[lane]) : 0u;
    v4u w4[NI], x0[NI], x1[NI];
#pragma unroll
    for (int i = 0; i < NI; i++) {
        int o = (i * 64 + lane) * 16;
        o = o < span ? o : span - 16;
        const int br = o >= RS ? o - RS : o;
        w4[i] = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(wb + o));
        const v4u* xp = reinterpret_cast<const v4u*>(xq + (size_t)br * 2);
        x0[i] = xp[0];
        x1[i] = xp[1];
    }
#pragma unroll
    for (int i = 0; i < NI; i++)
        acc ^= w4[i].x ^ w4[i].y ^ w4[i].z ^ w4[i].w ^ x0[i].x ^ x0[i].y ^ x0[i].z ^ x0[i].w ^ x1[i].x ^ x1[i].y ^
               x1[i].z ^ x1[i].w;
    if (acc == 0x9E3779B9u) sink[wv] = acc;   // practically never: keeps the loads live
}

template <int M>
hipError_t launch_gemv_loads(const uint32_t* wq, const uint16_t* ws, const int8_t* xq, uint32_t* sink, int N, int K,
                             int waves, int full, int nrem, int S, size_t lds, bool hs, hipStream_t st) {
    const int grid = full + nrem * S;
    if (hs)
        hipLaunchKernelGGL((gemv_loads_k<M, 2, true>), dim3(grid), dim3(64 * waves), lds, st, wq, ws, xq, sink, N, K,
                           full, nrem, S);
    else
        hipLaunchKernelGGL((gemv_loads_k<M, 2, false>), dim3(grid), dim3(64 * waves), lds, st, wq, ws, xq, sink, N,
                           K, full, nrem, S);
    return hipGetLastError();
}

__global__ void empty_k() {}

// ---- scaled f8f6f4 MFMA rate: four independent accumulator chains per wave.
// 8 independent chains of the unscaled 16x16x128 FP8 MFMA per wave (the scale
// builtin with zero scales compiles to the unscaled instruction).
__global__ __launch_bounds__(512) void mfma_f8_16_k(float* __restrict__ sink, int iters, int seed) {
    v8i a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (seed * (i + 1) + (int)threadIdx.x) & 0x3f3f3f3f;
        b[i] = (seed ^ (i * 77 + (int)threadIdx.x)) & 0x0f0f0f0f;
    }
    v4f c[8];
#pragma unroll
    for (int j = 0; j < 8; j++) c[j] = v4f{0.f, 0.f, 0.f, 0.f};
    for (int it = 0; it < iters; it++) {
#pragma unroll
        for (int j = 0; j < 8; j++)
            c[j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4((j & 1) ? a : b, (j & 2) ? a : b, c[j], 0, 0,
                                                                    0, 0, 0, 0);
    }
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < 8; j++) s += c[j][0] + c[j][1] + c[j][2] + c[j][3];
    if (s == 1234.5f) sink[blockIdx.x] = s;
}

template <int FMT>
__global__ __launch_bounds__(512) void mfma_f8f6f4_k(float* __restrict__ sink, int iters, int seed) {
    v8i a, b;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a[i] = (seed * (i + 1) + (int)threadIdx.x) & 0x3f3f3f3f;   // finite codes in every format
        b[i] = (seed ^ (i * 77 + (int)threadIdx.x)) & 0x0f0f0f0f;
    }
    v16f c0 = {}, c1 = {}, c2 = {}, c3 = {};
    for (int it = 0; it < iters; it++) {
        c0 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, c0, FMT, FMT, 0, 127, 0, 127);
        c1 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, a, c1, FMT, FMT, 0, 127, 0, 127);
        c2 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, a, c2, FMT, FMT, 0, 127, 0, 127);
        c3 = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(b, b, c3, FMT, FMT, 0, 127, 0, 127);
    }
    float s = 0.f;
#pragma unroll
    for (int r = 0; r < 16; r++) s += c0[r] + c1[r] + c2[r] + c3[r];
    if (s == 1234.5f) sink[blockIdx.x] = s;
}

// ---- the prefill GEMM's unit skeleton (rt4p_gemm_unit): registers only.  Operands
// change with the unit index so that nothing is loop-invariant.
template <int VARIANT>
__global__ __launch_bounds__(512, 1) void gemm_unit_k(float* __restrict__ sink, int units, int seed) {
    const int t = (int)threadIdx.x;
    v4i a4 = {seed ^ t, t * 3, seed >> 2, t ^ 0x55};
    v4i b4 = {t * 7, seed, t ^ 0x3c, seed * 5};
    v8i a8, b8;
#pragma unroll
    for (int i = 0; i < 8; i++) {
        a8[i] = (seed * (i + 1) + t) & 0x3f3f3f3f;
        b8[i] = (seed ^ (i * 77 + t)) & 0x0f0f0f0f;
    }
    const v4h sa = __builtin_bit_cast(v4h, make_uint2(0x3F803F80u ^ (t & 0x100), 0x3F003F00u));
    const v4h sb = __builtin_bit_cast(v4h, make_uint2(0x3F803F80u, (uint32_t)t << 16));
    const v16f zf = {};
    const v16i zi = {};
    v16f facc[4] = {zf, zf, zf, zf};
    v16f S = zf, R[2] = {zf, zf};
    v16i I[2] = {zi, zi};
    const v32f z32 = {};
    v32f S2 = z32;   // variant 0: scale products of a row-tile pair
    const float saf = __uint_as_float(0x3F800000u ^ (t & 0x100)), sbf = __uint_as_float(0x3F000000u + t);
    for (int u = 0; u < units; u++) {
#pragma unroll
        for (int ii = 0; ii < 4; ii++) {
            const int p = ii & 1, f = (ii + 3) & 3;
            // operands distinct per row tile and unit: no MFMA of the unit may be
            // merged with another or hoisted out of the loop
            v4i a = a4;
            a[1] ^= u * 4 + ii;
            v8i a8u = a8;
            a8u[1] ^= (u * 4 + ii) & 0x0f0f0f0f;
            v4h sau = sa;
            sau[0] ^= (short)(u * 4 + ii);
            if (VARIANT == 0) {
                // the fold of row tile ii - 1 takes the high half of the pair buffer for
                // odd tiles, the low half for even ones (tiles 3 and 0 of the previous
                // unit / this one: high, then low after the (0, 1) products)
                const int hi = (ii & 1) ^ 1;
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    I[p] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b4, k ? I[p] : zi, 0, 0, 0);
#pragma unroll
                    for (int r = 4 * k; r < 4 * k + 4; r++) {
                        float v = fmaf((float)I[p ^ 1][r], hi ? S2[16 + r] : S2[r], facc[f][r]);
                        asm volatile("" : "+v"(v));
                        facc[f][r] = v;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                if (ii == 0 || ii == 2)
                    S2 = __builtin_amdgcn_mfma_f32_32x32x1f32(saf + (float)(u * 4 + ii), sbf, z32, 0, 0, 0);
            } else {
                R[p] = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(sb, sau, zf, 0, 0, 0);   // the bias
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    R[p] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a8u, b8, R[p], 0, 0, 0, 127, 0, 136);
#pragma unroll
                    for (int r = 4 * k; r < 4 * k + 4; r++) {
                        float v = fmaf(R[p ^ 1][r], S[r], facc[f][r]);
                        asm volatile("" : "+v"(v));
                        facc[f][r] = v;
                    }
                    __builtin_amdgcn_sched_barrier(0);
                }
                S = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(sau, sb, zf, 0, 0, 0);
            }
        }
    }
    float s = 0.f;
#pragma unroll
    for (int i = 0; i < 4; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) s += facc[i][r];
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

int rt4p_gemv_loads(const void* wq, const void* ws, const void* xq, const void* sa, void* sink, int rows, int N,
                    int K, int groups_per_wave, int waves, int k_splits, int cus, void* stream) {
    const int gpw = groups_per_wave;
    if (gpw == 0) {   // the one-row dot-product form: two rows per wave, `waves` per workgroup
        const int ni = (K + 1023) / 1024;
        if (!wq || !ws || !xq || !sa || !sink || rows != 1 || N < 1 || K % 256 || K > 8192 || waves < 1 ||
            waves > 4)
            return 1;
        const int nw = (N + 1) / 2, grid = (nw + waves - 1) / waves;
        const uint32_t* w = static_cast<const uint32_t*>(wq);
        const uint16_t* s = static_cast<const uint16_t*>(ws);
        const int8_t* x = static_cast<const int8_t*>(xq);
        const float* a = static_cast<const float*>(sa);
        uint32_t* k = static_cast<uint32_t*>(sink);
        hipStream_t st = (hipStream_t)stream;
        switch (ni) {
#define RT4P_DOT(NI) \
    case NI: hipLaunchKernelGGL(gemv_loads_dot_k<NI>, dim3(grid), dim3(64 * waves), 0, st, w, s, x, a, k, N, K); break;
            RT4P_DOT(1) RT4P_DOT(2) RT4P_DOT(3) RT4P_DOT(4) RT4P_DOT(5) RT4P_DOT(6) RT4P_DOT(7) RT4P_DOT(8)
#undef RT4P_DOT
            default: return 1;
        }
        return hipGetLastError() == hipSuccess ? 0 : 3;
    }
    if (!wq || !ws || !xq || !sink || rows < 1 || rows > 4 || N < 1 || (gpw != 2 && gpw != 4) || K < 128 * gpw ||
        K % (128 * gpw) || waves < 1 || waves > (gpw == 4 ? 8 : 16) || k_splits < 1 || cus < 1)
        return 1;
    // the GEMV's grid (gemv_split) and, for 2 groups per wave, its dynamic LDS (launch_one)
    const int ntiles = (N + 15) / 16, NG = K / 128, NC = NG / gpw;
    int full = ntiles / cus * cus, nrem = ntiles - full, S = k_splits;
    if (S == 1) {
        full = ntiles;
        nrem = 0;
    }
    const uint32_t* w = static_cast<const uint32_t*>(wq);
    const uint16_t* s = static_cast<const uint16_t*>(ws);
    const int8_t* x = static_cast<const int8_t*>(xq);
    uint32_t* k = static_cast<uint32_t*>(sink);
    hipStream_t st = (hipStream_t)stream;
    hipError_t e;
    if (gpw == 4) {
        const int grid = full + nrem * S;
#define RT4P_TL(MM) hipLaunchKernelGGL(gemv_loads_tl_k<MM>, dim3(grid), dim3(64 * waves), 0, st, w, s, x, k, N, K, full, nrem, S)
        switch (rows) {
            case 1: RT4P_TL(1); break;
            case 2: RT4P_TL(2); break;
            case 3: RT4P_TL(3); break;
            default: RT4P_TL(4); break;
        }
#undef RT4P_TL
        e = hipGetLastError();
        return e == hipSuccess ? 0 : 3;
    }
    const size_t lds = (size_t)waves * 16 * 2 * 2 + (size_t)waves * rows * 16 * 4 + (size_t)waves * rows * 2 * 128;
    const int per_wave = (NC + waves - 1) / waves;
    const bool hs = waves <= 4 && per_wave >= 3 && per_wave <= 8;
    switch (rows) {
        case 1: e = launch_gemv_loads<1>(w, s, x, k, N, K, waves, full, nrem, S, lds, hs, st); break;
        case 2: e = launch_gemv_loads<2>(w, s, x, k, N, K, waves, full, nrem, S, lds, hs, st); break;
        case 3: e = launch_gemv_loads<3>(w, s, x, k, N, K, waves, full, nrem, S, lds, hs, st); break;
        default: e = launch_gemv_loads<4>(w, s, x, k, N, K, waves, full, nrem, S, lds, hs, st); break;
    }
    return e == hipSuccess ? 0 : 3;
}

int rt4p_empty(int blocks, int threads, void* stream) {
    if (blocks < 1 || threads < 1 || threads > 1024) return 1;
    hipLaunchKernelGGL(empty_k, dim3(blocks), dim3(threads), 0, (hipStream_t)stream);
    return last() == hipSuccess ? 0 : 3;
}

int rt4p_mfma_f8_16x16(void* sink, int iters, int blocks, void* stream) {
    if (!sink || iters < 1 || blocks < 1) return 1;
    hipLaunchKernelGGL(mfma_f8_16_k, dim3(blocks), dim3(512), 0, (hipStream_t)stream, static_cast<float*>(sink),
                       iters, 12345);
    return last() == hipSuccess ? 0 : 3;
}

int rt4p_mfma_f8f6f4(void* sink, int fmt, int iters, int blocks, void* stream) {
    if (!sink || iters < 1 || blocks < 1) return 1;
    hipStream_t st = (hipStream_t)stream;
    float* s = static_cast<float*>(sink);
    switch (fmt) {
        case 0: hipLaunchKernelGGL(mfma_f8f6f4_k<0>, dim3(blocks), dim3(512), 0, st, s, iters, 12345); break;
        case 2: hipLaunchKernelGGL(mfma_f8f6f4_k<2>, dim3(blocks), dim3(512), 0, st, s, iters, 12345); break;
        case 4: hipLaunchKernelGGL(mfma_f8f6f4_k<4>, dim3(blocks), dim3(512), 0, st, s, iters, 12345); break;
        default: return 1;
    }
    return last() == hipSuccess ? 0 : 3;
}

int rt4p_gemm_unit(void* sink, int variant, int units, int blocks, void* stream) {
    if (!sink || units < 1 || blocks < 1) return 1;
    hipStream_t st = (hipStream_t)stream;
    float* s = static_cast<float*>(sink);
    if (variant == 0)
        hipLaunchKernelGGL(gemm_unit_k<0>, dim3(blocks), dim3(512), 0, st, s, units, 12345);
    else if (variant == 1)
        hipLaunchKernelGGL(gemm_unit_k<1>, dim3(blocks), dim3(512), 0, st, s, units, 12345);
    else
        return 1;
    return last() == hipSuccess ? 0 : 3;
}

int rt4p_valu_fma(void* sink, int iters, int blocks, void* stream) {
    if (!sink || iters < 1 || blocks < 1) return 1;
    hipLaunchKernelGGL(valu_fma_k, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (float*)sink, iters, 0.5f);
    return last() == hipSuccess ? 0 : 3;
}

}  // extern "C"
