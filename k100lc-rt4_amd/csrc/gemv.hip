// gemv.hip -- RT4 W4A8 decode GEMV for M = 1..4 rows on gfx950 matrix cores.
//
//   y[m][n] = Σ_g f16(ws[n][g]) * sa[m][g] * I[m][n][g],
//   I[m][n][g] = Σ_{k in group g} code[n][k] * xq[m][k]      (exact int32)
//
// Restates gemv_w4a8 (kernels/gemv_w4a8_core.h:76-209) as called by k_gemv_w4a8
// (src/k_gemv.hip:53-106), redesigned for CDNA4:
//
// * The group dot products run on v_mfma_i32_16x16x64_i8.  A = the M activation
//   rows (rows M..15 of the 16-row operand are zero), B = 16 weight rows.  One
//   group (128 k) of a 16-row tile is exactly two MFMAs, and the int32
//   accumulator then holds 16*I exactly (the x16 nibble unpack, rt4_dev.h).
//   The MFMA pipe is ~10% busy at HBM speed and the VALU only unpacks
//   (3 ops/dword) and folds once per group, so the kernel is bound by HBM.
// * Lane l of a wave loads 16 contiguous bytes of weight row (n0 + l%16), quarter
//   l/16 of the group: one dwordx4 per lane covers 16 rows x 64 B.
// * A workgroup owns a tile of 16*RT rows; its `waves` waves split the K groups
//   of that tile and each issues all of its weight loads (<= 10 groups) before
//   touching anything else, so a CU keeps tens of KB of weight reads in flight.
// * The activations (M*K bytes, interleaved int8) are staged once per
//   workgroup in LDS; the partial sums of the waves are reduced through LDS.
// * The fp32 scale is applied once per group: the per-group term
//   fp32(16I) * (f16(ws)/16 * sa) equals the reference's (ws*sa)*I bit for bit
//   (power-of-two scaling is exact); only the order of the sum over groups
//   differs from the reference.
#include "rt4_dev.h"
#include "rt4_internal.h"

namespace rt4 {

// Two-tile workgroups keep twice the weight loads in flight per wave, so they
// are limited to 8 waves (2 waves per SIMD, up to 256 VGPRs each).
template <int RT>
constexpr int gemv_max_threads() { return RT == 1 ? 1024 : 512; }

template <int M, int RT, bool GSUM>
__global__ __launch_bounds__(gemv_max_threads<RT>()) void gemv_w4a8_k(const uint32_t* __restrict__ wq,
                                                    const uint16_t* __restrict__ ws,
                                                    const int8_t* __restrict__ xq,
                                                    const float* __restrict__ sa,
                                                    float* __restrict__ y,
                                                    int32_t* __restrict__ gsum, int N, int K) {
    constexpr int U = kGemvMaxGroupsPerWave;
    extern __shared__ __align__(16) unsigned char smem[];
    const int W = blockDim.x >> 6;
    const int lane = threadIdx.x & 63;
    const int w = uniform(threadIdx.x >> 6);
    const int col = lane & 15;  // weight row within a 16-row tile; activation row for A
    const int kb = lane >> 4;   // quarter of the 128-element group
    const int NG = K >> 7, KD = K >> 3;
    const int n0 = blockIdx.x * (16 * RT);
    const int g0 = uniform((int)(((long long)w * NG) / W));
    const int g1 = uniform((int)(((long long)(w + 1) * NG) / W));

    const uint4* wp[RT];
    const uint16_t* sp[RT];
#pragma unroll
    for (int t = 0; t < RT; t++) {
        int n = n0 + 16 * t + col;
        n = n < N ? n : N - 1;  // tail rows read a valid row; their results are dropped
        wp[t] = reinterpret_cast<const uint4*>(wq + (size_t)n * KD) + kb;
        sp[t] = ws + (size_t)n * NG;
    }

    // Stage the activations: read them into registers first, so that the weight
    // loads issued next are not held up behind them.
    const int n16 = (M * K) >> 4;
    constexpr int kStage = 4;  // uint4 per thread per pass (covers M*K <= 64*blockDim bytes per pass)
    const uint4* asrc = reinterpret_cast<const uint4*>(xq);
    uint4* adst = reinterpret_cast<uint4*>(smem);

    uint4 wv[U][RT];
    uint16_t swv[U][RT];
    float yacc[RT][M];
#pragma unroll
    for (int t = 0; t < RT; t++)
#pragma unroll
        for (int r = 0; r < M; r++) yacc[t][r] = 0.f;

    for (int base = 0; base < n16; base += kStage * (int)blockDim.x) {
        uint4 st[kStage];
#pragma unroll
        for (int j = 0; j < kStage; j++) {
            const int i = base + j * (int)blockDim.x + (int)threadIdx.x;
            if (i < n16) st[j] = asrc[i];
        }
        if (base == 0) {
            // first chunk of this wave's weights goes out while the stage loads fly
#pragma unroll
            for (int u = 0; u < U; u++)
                if (g0 + u < g1)
#pragma unroll
                    for (int t = 0; t < RT; t++) {
                        wv[u][t] = wp[t][(size_t)(g0 + u) * 4];
                        swv[u][t] = sp[t][g0 + u];
                    }
        }
#pragma unroll
        for (int j = 0; j < kStage; j++) {
            const int i = base + j * (int)blockDim.x + (int)threadIdx.x;
            if (i < n16) adst[i] = st[j];
        }
    }
    __syncthreads();

    const bool act = col < M;
    const uint4* arow = reinterpret_cast<const uint4*>(smem + (size_t)(act ? col : 0) * K) + 2 * kb;
    const v4i zero = {0, 0, 0, 0};

    for (int gc = g0; gc < g1; gc += U) {
        if (gc != g0) {
#pragma unroll
            for (int u = 0; u < U; u++)
                if (gc + u < g1)
#pragma unroll
                    for (int t = 0; t < RT; t++) {
                        wv[u][t] = wp[t][(size_t)(gc + u) * 4];
                        swv[u][t] = sp[t][gc + u];
                    }
        }
#pragma unroll
        for (int u = 0; u < U; u++) {
            const int g = gc + u;
            if (g < g1) {
                v4i a0 = zero, a1 = zero;
                if (act) {
                    const uint4 x0 = arow[(size_t)g * 8], x1 = arow[(size_t)g * 8 + 1];
                    a0 = v4i{(int)x0.x, (int)x0.y, (int)x0.z, (int)x0.w};
                    a1 = v4i{(int)x1.x, (int)x1.y, (int)x1.z, (int)x1.w};
                }
                float sav[M];
#pragma unroll
                for (int r = 0; r < M; r++) sav[r] = sa[(size_t)r * NG + g];
#pragma unroll
                for (int t = 0; t < RT; t++) {
                    const uint4 q = wv[u][t];
                    const v4i b0 = {(int)even_x16(q.x), (int)odd_x16(q.x), (int)even_x16(q.y),
                                    (int)odd_x16(q.y)};
                    const v4i b1 = {(int)even_x16(q.z), (int)odd_x16(q.z), (int)even_x16(q.w),
                                    (int)odd_x16(q.w)};
                    v4i acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0, b0, zero, 0, 0, 0);
                    acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1, b1, acc, 0, 0, 0);
                    // lane l < 16 now holds 16*I[m=r][n0+16t+l] in acc[r]
                    if (GSUM && lane < 16) {
                        const int n = n0 + 16 * t + lane;
                        if (n < N)
#pragma unroll
                            for (int r = 0; r < M; r++)
                                gsum[((size_t)r * N + n) * NG + g] = acc[r] >> 4;
                    }
                    const float s16 = f16_bits_to_f32(swv[u][t]) * 0.0625f;
#pragma unroll
                    for (int r = 0; r < M; r++)
                        yacc[t][r] = fmaf((float)acc[r], s16 * sav[r], yacc[t][r]);
                }
            }
        }
    }

    // Reduce the waves' partial sums (lanes 0..15 hold rows n0+16t+lane).
    __syncthreads();
    float* red = reinterpret_cast<float*>(smem);  // [W][RT][M][16]
    if (lane < 16)
#pragma unroll
        for (int t = 0; t < RT; t++)
#pragma unroll
            for (int r = 0; r < M; r++) red[((w * RT + t) * M + r) * 16 + lane] = yacc[t][r];
    __syncthreads();
    for (int i = threadIdx.x; i < RT * M * 16; i += blockDim.x) {
        const int c = i & 15, r = (i >> 4) % M, t = (i >> 4) / M;
        float s = 0.f;
        for (int v = 0; v < W; v++) s += red[((v * RT + t) * M + r) * 16 + c];
        const int n = n0 + 16 * t + c;
        if (n < N) y[(size_t)r * N + n] = s;
    }
}

GemvCfg gemv_default_cfg(int rows, int N, int K) {
    (void)rows;
    const int NG = K / kGroup;
    GemvCfg c;
    c.rt = (N >= 16384 && NG <= 8 * 5) ? 2 : 1;
    int w = (NG + 4) / 5;  // about five groups per wave
    const int maxw = (c.rt == 1 ? gemv_max_threads<1>() : gemv_max_threads<2>()) / 64;
    if (w < 1) w = 1;
    if (w > maxw) w = maxw;
    c.waves = w;
    return c;
}

bool gemv_cfg_valid(const GemvCfg& c, int K) {
    if (c.rt != 1 && c.rt != 2) return false;
    const int maxw = (c.rt == 1 ? gemv_max_threads<1>() : gemv_max_threads<2>()) / 64;
    return c.waves >= 1 && c.waves <= maxw && K > 0;
}

static size_t gemv_smem_bytes(int M, int K, const GemvCfg& c) {
    const size_t act = (size_t)M * K;
    const size_t red = (size_t)c.waves * c.rt * M * 16 * sizeof(float);
    return act > red ? act : red;
}

template <int M, int RT, bool GSUM>
static hipError_t launch_one(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws,
                             const int8_t* xq, const float* sa, int N, int K, int waves,
                             hipStream_t st) {
    const size_t smem = gemv_smem_bytes(M, K, GemvCfg{RT, waves});
    const void* fn = reinterpret_cast<const void*>(&gemv_w4a8_k<M, RT, GSUM>);
    if (smem > 65536) {
        static bool raised = false;  // per instantiation; attribute is per function
        if (!raised) {
            const hipError_t e =
                hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            if (e != hipSuccess) return e;
            raised = true;
        }
    }
    const dim3 grid((N + 16 * RT - 1) / (16 * RT));
    hipLaunchKernelGGL((gemv_w4a8_k<M, RT, GSUM>), grid, dim3(64 * waves), smem, st, wq, ws, xq,
                       sa, y, gsum, N, K);
    return hipGetLastError();
}

template <int M, bool GSUM>
static hipError_t launch_m(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws,
                           const int8_t* xq, const float* sa, int N, int K, const GemvCfg& c,
                           hipStream_t st) {
    if (c.rt == 2) return launch_one<M, 2, GSUM>(y, gsum, wq, ws, xq, sa, N, K, c.waves, st);
    return launch_one<M, 1, GSUM>(y, gsum, wq, ws, xq, sa, N, K, c.waves, st);
}

hipError_t launch_gemv_w4a8(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws,
                            const int8_t* xq, const float* sa, int rows, int N, int K,
                            const GemvCfg& cfg, hipStream_t st) {
    if (gsum) {
        switch (rows) {
            case 1: return launch_m<1, true>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 2: return launch_m<2, true>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 3: return launch_m<3, true>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 4: return launch_m<4, true>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
        }
    } else {
        switch (rows) {
            case 1: return launch_m<1, false>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 2: return launch_m<2, false>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 3: return launch_m<3, false>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
            case 4: return launch_m<4, false>(y, gsum, wq, ws, xq, sa, N, K, cfg, st);
        }
    }
    return hipErrorInvalidValue;
}

}  // namespace rt4
