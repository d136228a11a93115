// attn_feed.hip -- the feeders of the int4-KV attention prefill, gfx950: the
// query quantizer and the K/V cache appends (restating src/k_new.hip:228-399).
// Formats of qq, qsc, kc, ksc, vc, vsc are those in the header of attn.hip.  These
// kernels are built with the default machine scheduler; attn.hip (the prefill
// kernels) is built with another one, measured faster there and slower here.
#include "rt4_dev.h"
#include "rt4_internal.h"

namespace rt4 {

namespace {

// int4 code of x / s (s = amax/7 or 1), same IEEE ops as the reference quantizers.
__device__ __forceinline__ uint32_t code4(float x, float s) {
    return (uint32_t)clampi((int)lrintf(x / s), -8, 7) & 0xFu;
}
// The codes of 8 values as one dword (value e in nibble e), x / s taken through
// the reciprocal when every scale of the wave allows it (bit-equal to code4).
__device__ __forceinline__ uint32_t codes8(const float* v, float s) {
    uint32_t w = 0;
    if (__all(recip_div_ok(s))) {
        const float y = 1.f / s;
#pragma unroll
        for (int e = 0; e < 8; e++) w |= ((uint32_t)clampi((int)lrintf(div_by_recip(v[e], s, y)), -8, 7) & 0xFu) << (4 * e);
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) w |= code4(v[e], s) << (4 * e);
    }
    return w;
}

}  // namespace

// ------------------------------------------------------------------ feeders --

// Q of all heads (restates attn_q_quant_k, src/k_new.hip:228-253): x f32 [T][H][D]
// -> qq [H][TP][D/8], qs [H][D/G][TP].  One lane per 8 elements; a G-group is GL =
// G/8 consecutive lanes.  Rows >= T are not written.
template <int GL, bool ALIGNED>
__global__ __launch_bounds__(256) void attn_q_quant_k(uint32_t* __restrict__ qq, float* __restrict__ qs,
                                                      const float* __restrict__ x, int T, int H, int D, int TP) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int dw = D >> 3;
    if (i >= (size_t)T * H * dw) return;          // whole groups exit together
    const int e8 = (int)(i % dw);
    const int rh = (int)(i / dw), h = rh % H, r = rh / H;
    const float* xr = x + (size_t)rh * D + 8 * e8;  // (r*H + h)*D
    float v[8], amax = 0.f;
    if (ALIGNED) {
        const float4 a = reinterpret_cast<const float4*>(xr)[0], b = reinterpret_cast<const float4*>(xr)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = xr[e];
    }
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    amax = run_max<GL>(amax);
    const float s = amax > 0.f ? amax / 7.f : 1.f;
    const uint32_t w = codes8(v, s);
    qq[((size_t)h * TP + r) * dw + e8] = w;
    const int ng = D / (8 * GL);
    if (e8 % GL == 0) qs[((size_t)h * ng + e8 / GL) * TP + r] = s;
}

// K cache append (restates kv_append_k_k, src/k_new.hip:327-347): kf f32 [T][H][D]
// -> kc [H][kv_total][D/8], ksc [H][D/G][kv_total] at keys t0..t0+T-1.
template <int GL>
__global__ __launch_bounds__(256) void kv_append_k_k(uint32_t* __restrict__ kc, float* __restrict__ ksc,
                                                     const float* __restrict__ kf, int t0, int T, int H, int D,
                                                     int kv_total) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    const int dw = D >> 3;
    if (i >= (size_t)T * H * dw) return;
    const int e8 = (int)(i % dw);
    const int th = (int)(i / dw), h = th % H, t = th / H;
    const int kv = t0 + t;
    const float* xr = kf + (size_t)th * D + 8 * e8;
    float v[8], amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        v[e] = xr[e];
        amax = fmaxf(amax, fabsf(v[e]));
    }
    amax = run_max<GL>(amax);
    const float s = amax > 0.f ? amax / 7.f : 1.f;
    kc[((size_t)h * kv_total + kv) * dw + e8] = codes8(v, s);
    const int ng = D / (8 * GL);
    if (e8 % GL == 0) ksc[((size_t)h * ng + e8 / GL) * kv_total + kv] = s;
}

// V cache append (restates kv_append_v_k, src/k_new.hip:351-392).  The reference
// walks the 64-key tiles an append touches with one thread per (head, dim): new
// values go into the fp32 stage [H][BG][D] (the current partial tile), each tile
// is re-quantized from its valid slots (scale amax/7 per (tile, dim)), slots past
// the last valid one get code 0.  Every tile but the first of an append depends
// only on the new values, so here the tiles run in parallel (phase 1: one
// workgroup per (head, 64 dims, tile)), the first tile reading the stage's
// earlier slots; phase 2 then leaves the stage exactly as the sequential walk
// would (the last tile's values, and beneath them those of the tile before it).
// Phase 1 writes no stage slot, so the two phases are ordered by the stream.
__global__ __launch_bounds__(64) void kv_append_v_k(uint32_t* __restrict__ vc, float* __restrict__ vsc,
                                                    const float* __restrict__ stage, const float* __restrict__ vf,
                                                    int t0, int T, int H, int D, int BG, int kv_total) {
    const int h = blockIdx.x, d = blockIdx.y * 64 + threadIdx.x, ti = blockIdx.z;
    if (d >= D) return;
    const int first = t0 / BG, tile = first + ti, slot0 = ti == 0 ? t0 % BG : 0;
    const int done = ti == 0 ? 0 : (BG - t0 % BG) + (ti - 1) * BG;  // new values before this tile
    const int n = (T - done < BG - slot0) ? (T - done) : (BG - slot0);
    const int nval = slot0 + n;
    const float* st = stage + (size_t)h * BG * D + d;
    const float* src = vf + ((size_t)(done - slot0) * H + h) * D + d;  // slot i >= slot0 -> src[i*H*D]
    float amax = 0.f;
    for (int i = 0; i < nval; i++) {
        const float v = i < slot0 ? st[(size_t)i * D] : src[(size_t)i * H * D];
        amax = fmaxf(amax, fabsf(v));
    }
    const float s = amax > 0.f ? amax / 7.f : 1.f;
    vsc[((size_t)h * (kv_total / BG) + tile) * D + d] = s;
    uint32_t* out = vc + ((size_t)h * (kv_total / 8) + (size_t)tile * (BG / 8)) * D + d;
    for (int i = 0; i < BG; i += 8) {
        uint32_t w = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) {
            const int k = i + e;
            const float v = k < nval ? (k < slot0 ? st[(size_t)k * D] : src[(size_t)k * H * D]) : 0.f;
            w |= code4(v, s) << (4 * e);
        }
        out[(size_t)(i / 8) * D] = w;
    }
}

// Phase 2: the stage after the append.  Slot k holds the value of the last tile
// this append wrote it in: the last tile for its slots [slot0, nval), the tile
// before it (when this append also wrote that one) for the slots above nval,
// earlier content otherwise.  grid (H, D/64), 64 threads.
__global__ __launch_bounds__(64) void kv_stage_v_k(float* __restrict__ stage, const float* __restrict__ vf, int t0,
                                                   int T, int H, int D, int BG) {
    const int h = blockIdx.x, d = blockIdx.y * 64 + threadIdx.x;
    if (d >= D) return;
    const int first = t0 / BG, last = (t0 + T - 1) / BG;
    const int nval = (t0 + T - 1) % BG + 1;
    const int lo_last = last == first ? t0 % BG : 0;
    const int lo_prev = last - 1 == first ? t0 % BG : 0;
    float* st = stage + (size_t)h * BG * D + d;
    for (int k = 0; k < BG; k++) {
        int tok = -1;  // index of the new value that ends up in slot k
        if (k >= lo_last && k < nval) tok = last * BG + k - t0;
        else if (k >= nval && last > first && k >= lo_prev) tok = (last - 1) * BG + k - t0;
        if (tok >= 0) st[(size_t)k * D] = vf[((size_t)tok * H + h) * D + d];
    }
}

// The same two phases for the attention kernels' V tile of BG = 64 keys, with
// 256 threads per (head, 64 dims, tile): wave p owns keys 16p..16p+15, so each
// lane loads its 16 values once (coalesced across dims), the four waves combine
// their maxima through LDS and each lane packs its two code dwords from
// registers.  Values, scale and codes are those of kv_append_v_k: the maximum
// of a set does not depend on the order it is taken in, and keys past the valid
// ones are 0 in both.
__global__ __launch_bounds__(256) void kv_append_v64_k(uint32_t* __restrict__ vc, float* __restrict__ vsc,
                                                       const float* __restrict__ stage,
                                                       const float* __restrict__ vf, int t0, int T, int H, int D,
                                                       int kv_total) {
    constexpr int BG = 64;
    __shared__ float red[4][64];
    const int lane = threadIdx.x & 63, p = threadIdx.x >> 6;
    const int h = blockIdx.x, d = blockIdx.y * 64 + lane, ti = blockIdx.z;
    const bool dv = d < D;
    const int first = t0 / BG, tile = first + ti, slot0 = ti == 0 ? t0 % BG : 0;
    const int done = ti == 0 ? 0 : (BG - t0 % BG) + (ti - 1) * BG;  // new values before this tile
    const int n = (T - done < BG - slot0) ? (T - done) : (BG - slot0);
    const int nval = slot0 + n;
    const float* st = stage + (size_t)h * BG * D + d;
    const float* src = vf + ((size_t)(done - slot0) * H + h) * D + d;  // slot i >= slot0 -> src[i*H*D]
    float v[16];
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int k = 16 * p + e;
        float x = 0.f;
        if (dv && k < nval) x = k < slot0 ? st[(size_t)k * D] : src[(size_t)k * H * D];
        v[e] = x;
        amax = fmaxf(amax, fabsf(x));
    }
    red[p][lane] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0][lane], red[1][lane]), fmaxf(red[2][lane], red[3][lane]));
    if (!dv) return;
    const float s = amax > 0.f ? amax / 7.f : 1.f;
    if (p == 0) vsc[((size_t)h * (kv_total / BG) + tile) * D + d] = s;
    uint32_t* out = vc + ((size_t)h * (kv_total / 8) + (size_t)tile * (BG / 8)) * D + d;
#pragma unroll
    for (int j = 0; j < 2; j++) out[(size_t)(2 * p + j) * D] = codes8(v + 8 * j, s);
}

// Phase 2 for BG = 64: wave p restores slots 16p..16p+15 (see kv_stage_v_k).
__global__ __launch_bounds__(256) void kv_stage_v64_k(float* __restrict__ stage, const float* __restrict__ vf,
                                                      int t0, int T, int H, int D) {
    constexpr int BG = 64;
    const int lane = threadIdx.x & 63, p = threadIdx.x >> 6;
    const int h = blockIdx.x, d = blockIdx.y * 64 + lane;
    if (d >= D) return;
    const int first = t0 / BG, last = (t0 + T - 1) / BG;
    const int nval = (t0 + T - 1) % BG + 1;
    const int lo_last = last == first ? t0 % BG : 0;
    const int lo_prev = last - 1 == first ? t0 % BG : 0;
    float* st = stage + (size_t)h * BG * D + d;
#pragma unroll
    for (int e = 0; e < 16; e++) {
        const int k = 16 * p + e;
        int tok = -1;  // index of the new value that ends up in slot k
        if (k >= lo_last && k < nval) tok = last * BG + k - t0;
        else if (k >= nval && last > first && k >= lo_prev) tok = (last - 1) * BG + k - t0;
        if (tok >= 0) st[(size_t)k * D] = vf[((size_t)tok * H + h) * D + d];
    }
}

// -------------------------------------------------------------- launchers --

hipError_t launch_attn_q_quant(uint32_t* qq, float* qs, const float* x, int T, int H, int D, int G, int TP,
                               hipStream_t st) {
    const size_t n = (size_t)T * H * (D / 8);
    if (n == 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256));
    // rows of D (a multiple of 8) floats: every lane's 8 elements are 32-byte aligned
    // when x is 16-byte aligned
    const bool al = ((uintptr_t)x & 15) == 0;
#define RT4_QQ(GLV)                                                                                        \
    if (al) hipLaunchKernelGGL((attn_q_quant_k<GLV, true>), grid, dim3(256), 0, st, qq, qs, x, T, H, D, TP); \
    else hipLaunchKernelGGL((attn_q_quant_k<GLV, false>), grid, dim3(256), 0, st, qq, qs, x, T, H, D, TP);
    switch (G / 8) {
        case 8: RT4_QQ(8) break;
        case 16: RT4_QQ(16) break;
        case 32: RT4_QQ(32) break;
        default: return hipErrorInvalidValue;
    }
#undef RT4_QQ
    return hipGetLastError();
}

hipError_t launch_kv_append_k(uint32_t* kc, float* ksc, const float* kf, int t0, int T, int H, int D, int G,
                              int kv_total, hipStream_t st) {
    const size_t n = (size_t)T * H * (D / 8);
    if (n == 0) return hipSuccess;
    const dim3 grid((unsigned)((n + 255) / 256));
    switch (G / 8) {
        case 8: hipLaunchKernelGGL(kv_append_k_k<8>, grid, dim3(256), 0, st, kc, ksc, kf, t0, T, H, D, kv_total); break;
        case 16: hipLaunchKernelGGL(kv_append_k_k<16>, grid, dim3(256), 0, st, kc, ksc, kf, t0, T, H, D, kv_total); break;
        case 32: hipLaunchKernelGGL(kv_append_k_k<32>, grid, dim3(256), 0, st, kc, ksc, kf, t0, T, H, D, kv_total); break;
        default: return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

hipError_t launch_kv_append_v(uint32_t* vc, float* vsc, float* stage, const float* vf, int t0, int T, int H,
                              int D, int BG, int kv_total, hipStream_t st) {
    if (T <= 0) return hipSuccess;
    const int ntile = (t0 + T - 1) / BG - t0 / BG + 1;
    if (BG == 64) {   // the attention kernels' V tile
        hipLaunchKernelGGL(kv_append_v64_k, dim3(H, (D + 63) / 64, ntile), dim3(256), 0, st, vc, vsc, stage, vf, t0,
                           T, H, D, kv_total);
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        hipLaunchKernelGGL(kv_stage_v64_k, dim3(H, (D + 63) / 64), dim3(256), 0, st, stage, vf, t0, T, H, D);
        return hipGetLastError();
    }
    hipLaunchKernelGGL(kv_append_v_k, dim3(H, (D + 63) / 64, ntile), dim3(64), 0, st, vc, vsc, stage, vf, t0, T, H,
                       D, BG, kv_total);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(kv_stage_v_k, dim3(H, (D + 63) / 64), dim3(64), 0, st, stage, vf, t0, T, H, D, BG);
    return hipGetLastError();
}

}  // namespace rt4
