// gemm.hip -- RT4 W4A8 prefill GEMM on gfx950 int8 matrix cores.
//
//   C[m][n] = Σ_g sa[g][m] * sb[g][n] * I[m][n][g],
//   I[m][n][g] = Σ_{k in group g} q8[m][k] * code[n][k]        (exact int32)
//
// with q8 the prefill activation codes (quant_rows_a8_k semantics, src/k_new.hip:
// 268-301: q8 = 16h + l), sa their per-(group, row) scale (`sc`), code the RT4 int4
// weights and sb the fp32 group-major weight scales (src/model.cpp:190-202).
//
// The reference computes this as two int4 x int4 passes over the digit planes h
// and l plus an add (k_gemm_i4_a8, src/k_gemm.hip:22-34; kernel gemm_w4a4,
// kernels/gemm_core.h:59-206).  Per group its integer content is
// 16*I_h + I_l = I exactly, so here the digits are recombined into int8 once
// and a single int8 contraction runs on v_mfma_i32_32x32x32_i8:
//
// * Workgroup tile 128 activation rows x 256 weight rows, 8 waves, each wave a
//   64 x 64 block = 2 x 2 MFMA tiles of 32 x 32.  One 128-wide K group is four
//   MFMA k-steps; the int32 accumulators are restarted at every group (srcC = 0)
//   and folded into fp32 with one fma per output:  facc += f32(acc) * (sa/16 * sb).
//   acc holds 16*I exactly (the x16 nibble unpack, rt4_dev.h), the 1/16 is folded
//   into the staged activation scale (a power of two, so exact).
// * Per group the workgroup stages the int8 activation tile (128 x 128 B) and the
//   weight tile (256 rows x 64 B packed, unpacked once to 256 x 128 B of x16
//   bytes) in LDS, double-buffered: the global loads for group g+1 are issued
//   before the MFMAs of group g and land in LDS after them, one barrier per group.
//   LDS rows are padded to 144 B so the 16-byte fragment reads of 8 consecutive
//   lanes (8 consecutive rows) hit 32 distinct banks.
// * Rows past M or N read a clamped (valid) row; their outputs are not stored.
#include "rt4_dev.h"
#include "rt4_internal.h"

namespace rt4 {

namespace {

constexpr int BM = 128;           // activation rows per workgroup
constexpr int BN = 256;           // weight rows (output columns) per workgroup
constexpr int NT = 512;           // 8 waves
constexpr int LROW = 144;         // LDS bytes per staged row (128 + 16 pad)
constexpr int A_BYTES = BM * LROW;
constexpr int B_BYTES = BN * LROW;
constexpr int STAGE = A_BYTES + B_BYTES + (BM + BN) * 4;
constexpr size_t GEMM_LDS = 2 * (size_t)STAGE;

struct Prefetch {
    uint4 a[2];    // 2 x 16 B of int8 activations
    uint4 b[2];    // 2 x 16 B of packed weights (32 codes each)
    float s;       // one activation or weight scale
};

__device__ __forceinline__ void gemm_load(Prefetch& p, const int8_t* __restrict__ A,
                                          const uint32_t* __restrict__ W,
                                          const float* __restrict__ sa,
                                          const float* __restrict__ sb, int M, int N, int K,
                                          int bm, int bn, int g) {
    const int t = threadIdx.x;
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int id = t + j * NT;
        int r = bm + (id >> 3);
        r = r < M ? r : M - 1;
        p.a[j] = *reinterpret_cast<const uint4*>(A + (size_t)r * K + (size_t)g * 128 + (id & 7) * 16);
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int id = t + j * NT;
        int r = bn + (id >> 2);
        r = r < N ? r : N - 1;
        p.b[j] = *reinterpret_cast<const uint4*>(W + (size_t)r * (K >> 3) + (size_t)g * 16 + (id & 3) * 4);
    }
    if (t < BM) {
        int r = bm + t;
        r = r < M ? r : M - 1;
        p.s = sa[(size_t)g * M + r];
    } else if (t < BM + BN) {
        int r = bn + t - BM;
        r = r < N ? r : N - 1;
        p.s = sb[(size_t)g * N + r];
    }
}

__device__ __forceinline__ void gemm_store(const Prefetch& p, unsigned char* stage) {
    const int t = threadIdx.x;
    unsigned char* la = stage;
    unsigned char* lb = stage + A_BYTES;
    float* ls = reinterpret_cast<float*>(stage + A_BYTES + B_BYTES);
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int id = t + j * NT;
        *reinterpret_cast<uint4*>(la + (id >> 3) * LROW + (id & 7) * 16) = p.a[j];
    }
#pragma unroll
    for (int j = 0; j < 2; j++) {
        const int id = t + j * NT;
        const uint4 q = p.b[j];
        unsigned char* dst = lb + (id >> 2) * LROW + (id & 3) * 32;
        *reinterpret_cast<uint4*>(dst) = make_uint4(even_x16(q.x), odd_x16(q.x), even_x16(q.y), odd_x16(q.y));
        *reinterpret_cast<uint4*>(dst + 16) =
            make_uint4(even_x16(q.z), odd_x16(q.z), even_x16(q.w), odd_x16(q.w));
    }
    if (t < BM)
        ls[t] = p.s * 0.0625f;  // activation scale / 16 (undoes the x16 weight unpack, exact)
    else if (t < BM + BN)
        ls[t] = p.s;
}

template <bool GSUM>
__global__ __launch_bounds__(NT, 1) void gemm_w4a8_k(const int8_t* __restrict__ A,
                                                     const uint32_t* __restrict__ W,
                                                     const float* __restrict__ sa,
                                                     const float* __restrict__ sb,
                                                     float* __restrict__ C,
                                                     int32_t* __restrict__ gsum, int M, int N,
                                                     int K) {
    extern __shared__ __align__(16) unsigned char smem[];
    const int lane = threadIdx.x & 63;
    const int w = uniform(threadIdx.x >> 6);
    const int wm = w & 1, wn = w >> 1;
    const int bm = blockIdx.y * BM, bn = blockIdx.x * BN;
    const int NG = K >> 7;
    const int lr = lane & 31, lh = lane >> 5;

    v16i facc[2][2];
#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++)
#pragma unroll
            for (int r = 0; r < 16; r++) facc[i][j][r] = 0;  // bit pattern of +0.0f
    Prefetch pf;
    gemm_load(pf, A, W, sa, sb, M, N, K, bm, bn, 0);
    gemm_store(pf, smem);
    __syncthreads();

    const v16i zero16 = {};
    for (int g = 0; g < NG; g++) {
        unsigned char* cur = smem + (size_t)(g & 1) * STAGE;
        if (g + 1 < NG) gemm_load(pf, A, W, sa, sb, M, N, K, bm, bn, g + 1);

        const unsigned char* la = cur + (64 * wm + lr) * LROW + lh * 16;
        const unsigned char* lb = cur + A_BYTES + (64 * wn + lr) * LROW + lh * 16;
        v16i acc[2][2];
#pragma unroll
        for (int ks = 0; ks < 4; ks++) {
            v4i a[2], b[2];
#pragma unroll
            for (int i = 0; i < 2; i++) a[i] = *reinterpret_cast<const v4i*>(la + i * 32 * LROW + ks * 32);
#pragma unroll
            for (int j = 0; j < 2; j++) b[j] = *reinterpret_cast<const v4i*>(lb + j * 32 * LROW + ks * 32);
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a[i], b[j], ks == 0 ? zero16 : acc[i][j],
                                                                      0, 0, 0);
        }

        // fold: lane holds column n = 32j + lr, rows 8q + 4lh + e (q, e = 0..3) of tile (i, j)
        const float* ls = reinterpret_cast<const float*>(cur + A_BYTES + B_BYTES);
        float sbv[2];
#pragma unroll
        for (int j = 0; j < 2; j++) sbv[j] = ls[BM + 64 * wn + 32 * j + lr];
#pragma unroll
        for (int i = 0; i < 2; i++) {
            float sav[16];
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const float4 v = *reinterpret_cast<const float4*>(ls + 64 * wm + 32 * i + 8 * q + 4 * lh);
                sav[4 * q + 0] = v.x;
                sav[4 * q + 1] = v.y;
                sav[4 * q + 2] = v.z;
                sav[4 * q + 3] = v.w;
            }
#pragma unroll
            for (int j = 0; j < 2; j++)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const float f = __int_as_float(facc[i][j][r]);
                    facc[i][j][r] = __float_as_int(fmaf((float)acc[i][j][r], sav[r] * sbv[j], f));
                }
        }
        if (GSUM) {
#pragma unroll
            for (int i = 0; i < 2; i++)
#pragma unroll
                for (int j = 0; j < 2; j++) {
                    const int n = bn + 64 * wn + 32 * j + lr;
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int m = bm + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                        if (m < M && n < N) gsum[((size_t)m * N + n) * NG + g] = acc[i][j][r] >> 4;
                    }
                }
        }

        if (g + 1 < NG) gemm_store(pf, smem + (size_t)((g + 1) & 1) * STAGE);
        __syncthreads();
    }

#pragma unroll
    for (int i = 0; i < 2; i++)
#pragma unroll
        for (int j = 0; j < 2; j++) {
            const int n = bn + 64 * wn + 32 * j + lr;
            if (n < N)
#pragma unroll
                for (int r = 0; r < 16; r++) {
                    const int m = bm + 64 * wm + 32 * i + 8 * (r >> 2) + 4 * lh + (r & 3);
                    if (m < M) C[(size_t)m * N + n] = __int_as_float(facc[i][j][r]);
                }
        }
}

template <bool GSUM>
hipError_t launch_gemm_t(float* C, int32_t* gsum, const int8_t* A, const uint32_t* W,
                         const float* sa, const float* sb, int M, int N, int K, hipStream_t st) {
    static bool raised = false;  // the attribute is per function; set once
    if (!raised) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemm_w4a8_k<GSUM>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, (int)GEMM_LDS);
        if (e != hipSuccess) return e;
        raised = true;
    }
    const dim3 grid((N + BN - 1) / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL(gemm_w4a8_k<GSUM>, grid, dim3(NT), GEMM_LDS, st, A, W, sa, sb, C, gsum, M, N, K);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_w4a8(float* C, int32_t* gsum, const int8_t* A, const uint32_t* W,
                            const float* sa, const float* sb, int M, int N, int K, hipStream_t st) {
    if (gsum) return launch_gemm_t<true>(C, gsum, A, W, sa, sb, M, N, K, st);
    return launch_gemm_t<false>(C, gsum, A, W, sa, sb, M, N, K, st);
}

}  // namespace rt4
