// quant.hip -- activation quantizers of the RT4 path, gfx950.
//
// Three reference quantizers are restated here; each must produce bit-identical
// integer codes and scales, so every step computes the same IEEE single results
// as the reference: the correctly rounded quotient x/s (hipcc's division, or the
// reciprocal form of rt4_dev.h's div_by_recip, which equals it wherever a wave
// takes it) and round-half-to-even lrintf.  One lane owns 8 consecutive elements of a row,
// so a G-element group is an aligned run of G/8 lanes and its max-abs is a
// short xor-shuffle reduction; loads and stores are full dwords.
#include "rt4_dev.h"
#include "rt4_internal.h"

namespace rt4 {

// Load 8 consecutive floats; vector loads when the address is 16-byte aligned.
__device__ __forceinline__ void load8(const float* p, bool aligned, float v[8]) {
    if (aligned) {
        const float4 a = reinterpret_cast<const float4*>(p)[0];
        const float4 b = reinterpret_cast<const float4*>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) v[e] = p[e];
    }
}

// Eight int8 codes -> two dwords in the interleaved order [c0 c2 c4 c6 | c1 c3 c5 c7].
__device__ __forceinline__ uint2 interleave8(const int c[8]) {
    uint2 r;
    r.x = (uint32_t)(c[0] & 0xFF) | (uint32_t)(c[2] & 0xFF) << 8 | (uint32_t)(c[4] & 0xFF) << 16 |
          (uint32_t)(c[6] & 0xFF) << 24;
    r.y = (uint32_t)(c[1] & 0xFF) | (uint32_t)(c[3] & 0xFF) << 8 | (uint32_t)(c[5] & 0xFF) << 16 |
          (uint32_t)(c[7] & 0xFF) << 24;
    return r;
}

// ---------------------------------------------------------------------------
// Decode-side quantizer (restates quant_act, kernels/gemv_w4a8_core.h:34-66):
// per (row, 128-group) s = amax>0 ? amax/127 : 1, q = clamp(lrintf(x/s), -128, 127).
// Outputs: xq int8 [rows][K] interleaved, sa f32 [rows][K/128], and optionally
// asu = Σq per group (the reference needs it for its u=code+8 correction; the
// MFMA GEMV here does not, but it is kept for parity checks).
// x/s: for a wave whose scales all lie in [2^-96, 2^100], rt4_dev.h's
// div_by_recip (a correctly rounded reciprocal y = 1/s and one fused correction
// step, equal to the IEEE quotient on every targeted input checked, see there);
// other waves (tiny or non-finite groups) divide.
// ALIGNED: x rows 16-byte aligned (vector loads); SUMS: asu is written.
// grid (ceil(K/8/256), rows), block 256.
template <bool ALIGNED, bool SUMS>
__global__ __launch_bounds__(256) void quant_act_a8_k(const float* __restrict__ x,
                                                      int8_t* __restrict__ xq,
                                                      float* __restrict__ sa,
                                                      int32_t* __restrict__ asu, int K) {
    const int m = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;  // 8-element block in the row
    if (i >= (K >> 3)) return;                     // K%128==0: whole 16-lane runs exit together
    float v[8];
    load8(x + (size_t)m * K + 8 * (size_t)i, ALIGNED, v);
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    amax = run_max<16>(amax);
    const float s = amax > 0.f ? amax / 127.f : 1.f;
    int c[8];
    if (__all(recip_div_ok(s))) {
        const float y = 1.f / s;
#pragma unroll
        for (int e = 0; e < 8; e++) c[e] = clampi((int)lrintf(div_by_recip(v[e], s, y)), -128, 127);
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) c[e] = clampi((int)lrintf(v[e] / s), -128, 127);
    }
    *reinterpret_cast<uint2*>(xq + (size_t)m * K + 8 * (size_t)i) = interleave8(c);
    const int NG = K >> 7;
    if ((i & 15) == 0) sa[(size_t)m * NG + (i >> 4)] = s;
    if constexpr (SUMS) {
        int part = 0;
#pragma unroll
        for (int e = 0; e < 8; e++) part += c[e];
        part = run_sum<16>(part);
        if ((i & 15) == 0) asu[(size_t)m * NG + (i >> 4)] = part;
    }
}

hipError_t launch_quant_act_a8(int8_t* xq, float* sa, int32_t* asu, const float* x, int rows,
                               int K, hipStream_t st) {
    const dim3 grid((K / 8 + 255) / 256, rows);
    const bool aligned = ((uintptr_t)x & 15) == 0;
    if (aligned && !asu)
        hipLaunchKernelGGL((quant_act_a8_k<true, false>), grid, dim3(256), 0, st, x, xq, sa, asu, K);
    else if (aligned)
        hipLaunchKernelGGL((quant_act_a8_k<true, true>), grid, dim3(256), 0, st, x, xq, sa, asu, K);
    else if (!asu)
        hipLaunchKernelGGL((quant_act_a8_k<false, false>), grid, dim3(256), 0, st, x, xq, sa, asu, K);
    else
        hipLaunchKernelGGL((quant_act_a8_k<false, true>), grid, dim3(256), 0, st, x, xq, sa, asu, K);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Per-row activation quantizer (G = K: one scale per row).  An opt-in mode with no
// counterpart in the reference, which quantizes per (row, 128-group): the steps of
// quant_act_a8_k (DIV 127, codes in [-128, 127]) or of quant_rows_a8_k's int8 form
// (DIV 119, codes in [-128, 119]) with the row's max-abs, and the row's scale
// written into every 128-group slot of the per-group layout, so that the GEMV and
// the GEMM consume it unchanged (their fold multiplies s by the group's weight
// scale).  One workgroup per row: a pass over the row for its max-abs (a block
// reduction), then the quantization pass over the now cached row.  A lane handles
// 8-element blocks i = threadIdx.x + 256 j; K % 128 == 0 keeps the 16 blocks of a
// group on 16 consecutive lanes of one pass, all active or all not.
// GROUP_MAJOR: scales [K/128][rows] (the GEMM's), else [rows][K/128] (the GEMV's);
// asu (optional, [rows][K/128]): Σq per group.  grid (rows), block 256.
template <int DIV, bool ALIGNED, bool GROUP_MAJOR>
__global__ __launch_bounds__(256) void quant_row_k(const float* __restrict__ x, int8_t* __restrict__ xq,
                                                   float* __restrict__ sa, int32_t* __restrict__ asu, int rows,
                                                   int K) {
    __shared__ float red[4];
    const int m = blockIdx.x;
    const float* xr = x + (size_t)m * K;
    const int nb = K >> 3;
    float amax = 0.f;
    for (int i = threadIdx.x; i < nb; i += 256) {
        float v[8];
        load8(xr + 8 * (size_t)i, ALIGNED, v);
#pragma unroll
        for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    }
    amax = run_max<64>(amax);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float s = amax > 0.f ? amax / (float)DIV : 1.f;
    const bool by_recip = recip_div_ok(s);   // the same for the whole row
    const float y = 1.f / s;
    const int NG = K >> 7;
    for (int i = threadIdx.x; i < nb; i += 256) {
        float v[8];
        load8(xr + 8 * (size_t)i, ALIGNED, v);
        int c[8];
#pragma unroll
        for (int e = 0; e < 8; e++)
            c[e] = clampi((int)lrintf(by_recip ? div_by_recip(v[e], s, y) : v[e] / s), -128, DIV == 127 ? 127 : 119);
        *reinterpret_cast<uint2*>(xq + (size_t)m * K + 8 * (size_t)i) = interleave8(c);
        const int g = i >> 4;
        if ((i & 15) == 0) sa[GROUP_MAJOR ? (size_t)g * rows + m : (size_t)m * NG + g] = s;
        if (asu) {
            int part = 0;
#pragma unroll
            for (int e = 0; e < 8; e++) part += c[e];
            part = run_sum<16>(part);
            if ((i & 15) == 0) asu[(size_t)m * NG + g] = part;
        }
    }
}

hipError_t launch_quant_row(int8_t* xq, float* sa, int32_t* asu, const float* x, int rows, int K, int mode,
                            hipStream_t st) {
    const bool aligned = ((uintptr_t)x & 15) == 0;
    const dim3 grid(rows);
    if (mode == 0 && aligned)
        hipLaunchKernelGGL((quant_row_k<127, true, false>), grid, dim3(256), 0, st, x, xq, sa, asu, rows, K);
    else if (mode == 0)
        hipLaunchKernelGGL((quant_row_k<127, false, false>), grid, dim3(256), 0, st, x, xq, sa, asu, rows, K);
    else if (aligned)
        hipLaunchKernelGGL((quant_row_k<119, true, true>), grid, dim3(256), 0, st, x, xq, sa, asu, rows, K);
    else
        hipLaunchKernelGGL((quant_row_k<119, false, true>), grid, dim3(256), 0, st, x, xq, sa, asu, rows, K);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Prefill-side quantizer (restates quant_rows_a8_k, src/k_new.hip:268-301):
// per (row, G-group) s = amax>0 ? amax/119 : 1, q8 = clamp(lrintf(x/s), -128, 119),
// h = (q8+8)>>4, l = q8-16h.  Outputs the reference's layout: qh, ql u32
// [rows][K/8] nibble-packed like RT4 weights, sc and sc16 = 16*sc f32 group-major
// [K/G][rows].  Optionally also writes the int8 code q8 itself, interleaved
// [rows][K], which is what the MFMA GEMM consumes.
// GL = G/8 lanes per group.  grid (ceil(K/8/256), rows), block 256.
template <int GL>
__global__ __launch_bounds__(512) void quant_rows_a8_k(
    const float* __restrict__ x, uint32_t* __restrict__ qh, uint32_t* __restrict__ ql,
    float* __restrict__ sc, float* __restrict__ sc16, int8_t* __restrict__ xq, int rows, int K,
    int in_stride, int in_off, int x_aligned) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (K >> 3)) return;  // K%G==0: whole GL-lane runs exit together
    float v[8];
    load8(x + (size_t)r * in_stride + in_off + 8 * (size_t)i, x_aligned, v);
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    amax = run_max<GL>(amax);
    const float s = amax > 0.f ? amax / 119.f : 1.f;
    uint32_t wh = 0, wl = 0;
    int c[8];
    float qv[8];   // x / s: through the reciprocal when the wave's scales allow (bit-equal)
    if (__all(recip_div_ok(s))) {
        const float y = 1.f / s;
#pragma unroll
        for (int e = 0; e < 8; e++) qv[e] = div_by_recip(v[e], s, y);
    } else {
#pragma unroll
        for (int e = 0; e < 8; e++) qv[e] = v[e] / s;
    }
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int q8 = clampi((int)lrintf(qv[e]), -128, 119);
        const int h = (q8 + 8) >> 4;  // floor, also for negatives
        const int l = q8 - 16 * h;    // in [-8, 7]
        wh |= (uint32_t)(h & 0xF) << (4 * e);
        wl |= (uint32_t)(l & 0xF) << (4 * e);
        c[e] = q8;
    }
    const size_t d = (size_t)r * (K >> 3) + i;
    if (qh) qh[d] = wh;
    if (ql) ql[d] = wl;
    if (i % GL == 0) {
        const size_t gi = (size_t)(i / GL) * rows + r;
        if (sc) sc[gi] = s;
        if (sc16) sc16[gi] = s * 16.f;
    }
    if (xq) *reinterpret_cast<uint2*>(xq + (size_t)r * K + 8 * (size_t)i) = interleave8(c);
}

// int4 activation quantizer (restates quant_rows_k, src/k_new.hip:192-219):
// s = amax>0 ? amax/7 : 1, c = clamp(lrintf(x/s), -8, 7), nibble-packed, sc group-major.
template <int GL>
__global__ __launch_bounds__(512) void quant_rows_a4_k(const float* __restrict__ x,
                                                       uint32_t* __restrict__ q,
                                                       float* __restrict__ sc, int rows, int K,
                                                       int in_stride, int in_off, int x_aligned) {
    const int r = blockIdx.y;
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (K >> 3)) return;
    float v[8];
    load8(x + (size_t)r * in_stride + in_off + 8 * (size_t)i, x_aligned, v);
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    amax = run_max<GL>(amax);
    const float s = amax > 0.f ? amax / 7.f : 1.f;
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) {
        const int cc = clampi((int)lrintf(v[e] / s), -8, 7);
        w |= (uint32_t)(cc & 0xF) << (4 * e);
    }
    q[(size_t)r * (K >> 3) + i] = w;
    if (i % GL == 0) sc[(size_t)(i / GL) * rows + r] = s;
}

#define RT4_GL_CASES(KERNEL, ...)                                                         \
    switch (G / 8) {                                                                      \
        case 1: hipLaunchKernelGGL(KERNEL<1>, grid, dim3(bs), 0, st, __VA_ARGS__); break;  \
        case 2: hipLaunchKernelGGL(KERNEL<2>, grid, dim3(bs), 0, st, __VA_ARGS__); break;  \
        case 4: hipLaunchKernelGGL(KERNEL<4>, grid, dim3(bs), 0, st, __VA_ARGS__); break;  \
        case 8: hipLaunchKernelGGL(KERNEL<8>, grid, dim3(bs), 0, st, __VA_ARGS__); break;  \
        case 16: hipLaunchKernelGGL(KERNEL<16>, grid, dim3(bs), 0, st, __VA_ARGS__); break; \
        case 32: hipLaunchKernelGGL(KERNEL<32>, grid, dim3(bs), 0, st, __VA_ARGS__); break; \
        case 64: hipLaunchKernelGGL(KERNEL<64>, grid, dim3(bs), 0, st, __VA_ARGS__); break; \
        default: return hipErrorInvalidValue;                                             \
    }

bool quant_group_supported(int G) {
    return G >= 8 && G <= 512 && (G & (G - 1)) == 0;
}

// Lanes per workgroup for the row quantizers (one lane per 8 elements of a row,
// one grid row per input row): the largest multiple of 64 up to 512 that divides
// the K/8 lanes of a row, so that no workgroup is partly idle (K = 5120: 2 x 320
// lanes instead of 256 + 256 + 128); 256 with a partial last workgroup when K/8 is
// not a multiple of 64.  Multiples of 64 keep every G-group (at most 64 lanes)
// inside one wave.
int row_quant_lanes(int K) {
    const int kd = K / 8;
    for (int bs = 512; bs >= 64; bs -= 64)
        if (kd % bs == 0) return bs;
    return 256;
}

hipError_t launch_quant_rows_a8(uint32_t* qh, uint32_t* ql, float* sc, float* sc16, int8_t* xq,
                                const float* x, int rows, int K, int G, int in_stride, int in_off,
                                hipStream_t st) {
    if (in_stride == 0) in_stride = K;
    const int bs = row_quant_lanes(K);
    const dim3 grid((K / 8 + bs - 1) / bs, rows);
    const int aligned = (((uintptr_t)(x + in_off)) & 15) == 0 && (in_stride % 4) == 0;
    RT4_GL_CASES(quant_rows_a8_k, x, qh, ql, sc, sc16, xq, rows, K, in_stride, in_off, aligned);
    return hipGetLastError();
}

hipError_t launch_quant_rows_a4(uint32_t* q, float* sc, const float* x, int rows, int K, int G,
                                int in_stride, int in_off, hipStream_t st) {
    if (in_stride == 0) in_stride = K;
    const int bs = row_quant_lanes(K);
    const dim3 grid((K / 8 + bs - 1) / bs, rows);
    const int aligned = (((uintptr_t)(x + in_off)) & 15) == 0 && (in_stride % 4) == 0;
    RT4_GL_CASES(quant_rows_a4_k, x, q, sc, rows, K, in_stride, in_off, aligned);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// h/l digit planes -> int8 codes q8 = 16h + l, interleaved, for the MFMA GEMM.
// Bytewise: x = (h<<4) | (l^8) is q8+8 with no carries between bytes; the
// per-byte subtraction of 8 then uses the borrow-free SWAR form
// ((x | 0x80..) - 0x08..) ^ (~x & 0x80..).  One lane per dword pair.
__device__ __forceinline__ uint32_t swar_sub8(uint32_t x) {
    return ((x | 0x80808080u) - 0x08080808u) ^ (~x & 0x80808080u);
}

// One digit dword pair -> the 8 int8 codes of those 8 elements (interleaved order).
template <bool HAS_H>
__device__ __forceinline__ uint2 hl_pair(uint32_t h, uint32_t l) {
    if (!HAS_H) h = 0u;
    l ^= 0x88888888u;
    const uint32_t xe = ((h << 4) & 0xF0F0F0F0u) | (l & 0x0F0F0F0Fu);
    const uint32_t xo = (h & 0xF0F0F0F0u) | ((l >> 4) & 0x0F0F0F0Fu);
    return make_uint2(swar_sub8(xe), swar_sub8(xo));
}

// VEC: four dwords of each plane per lane (16-byte loads, two 16-byte stores; all
// three buffers 16-byte aligned), the last ndw % 4 dwords by the lane after the last
// whole quad; otherwise one dword per lane.
template <bool HAS_H, bool VEC>
__global__ __launch_bounds__(256) void hl_to_i8_k(const uint32_t* __restrict__ qh,
                                                  const uint32_t* __restrict__ ql,
                                                  int8_t* __restrict__ xq, size_t ndw) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if constexpr (VEC) {
        const size_t nq = ndw / 4;
        if (i < nq) {
            const uint4 l = reinterpret_cast<const uint4*>(ql)[i];
            const uint4 h = HAS_H ? reinterpret_cast<const uint4*>(qh)[i] : make_uint4(0, 0, 0, 0);
            const uint2 a = hl_pair<HAS_H>(h.x, l.x), b = hl_pair<HAS_H>(h.y, l.y);
            const uint2 c = hl_pair<HAS_H>(h.z, l.z), d = hl_pair<HAS_H>(h.w, l.w);
            uint4* o = reinterpret_cast<uint4*>(xq) + 2 * i;
            o[0] = make_uint4(a.x, a.y, b.x, b.y);
            o[1] = make_uint4(c.x, c.y, d.x, d.y);
        } else if (i == nq) {
            for (size_t j = 4 * nq; j < ndw; j++)
                reinterpret_cast<uint2*>(xq)[j] = hl_pair<HAS_H>(HAS_H ? qh[j] : 0u, ql[j]);
        }
    } else {
        if (i >= ndw) return;
        reinterpret_cast<uint2*>(xq)[i] = hl_pair<HAS_H>(HAS_H ? qh[i] : 0u, ql[i]);
    }
}

hipError_t launch_hl_to_i8(int8_t* xq, const uint32_t* qh, const uint32_t* ql, int rows, int K,
                           hipStream_t st) {
    const size_t ndw = (size_t)rows * (K / 8);
    const bool vec = ((uintptr_t)xq & 15) == 0 && ((uintptr_t)ql & 15) == 0 && ((uintptr_t)qh & 15) == 0;
    const unsigned blocks = (unsigned)(((vec ? ndw / 4 + 1 : ndw) + 255) / 256);
#define RT4_HL(H, V) hipLaunchKernelGGL((hl_to_i8_k<H, V>), dim3(blocks), dim3(256), 0, st, qh, ql, xq, ndw)
    if (qh) {
        if (vec) RT4_HL(true, true);
        else RT4_HL(true, false);
    } else {  // int4 codes alone (W4A4): sign-extended into the same interleaved int8 order
        if (vec) RT4_HL(false, true);
        else RT4_HL(false, false);
    }
#undef RT4_HL
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Decode int4 activation quantizer (restates quant_act4, kernels/gemv_w4a4_core.h:
// 22-44): per (row, 32-element subgroup) s = amax>0 ? amax/7 : 1,
// q = clamp(lrintf(x/s), -8, 7).  Outputs codes u32 [rows][K/8] in the RT4
// nibble order (low nibble = even k) and scales f32 [rows][K/32].  One lane per
// 8 elements (one output dword); a subgroup is 4 lanes.  grid (ceil(K/8/256), rows).
__global__ __launch_bounds__(256) void quant_act_a4_k(const float* __restrict__ x, uint32_t* __restrict__ aq,
                                                      float* __restrict__ sa, int K, int x_aligned) {
    const int m = blockIdx.y;
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= (K >> 3)) return;                     // K%32==0: whole 4-lane runs exit together
    float v[8];
    load8(x + (size_t)m * K + 8 * (size_t)i, x_aligned, v);
    float amax = 0.f;
#pragma unroll
    for (int e = 0; e < 8; e++) amax = fmaxf(amax, fabsf(v[e]));
    amax = run_max<4>(amax);
    const float s = amax > 0.f ? amax / 7.f : 1.f;
    uint32_t w = 0;
#pragma unroll
    for (int e = 0; e < 8; e++) w |= ((uint32_t)clampi((int)lrintf(v[e] / s), -8, 7) & 0xFu) << (4 * e);
    aq[(size_t)m * (K >> 3) + i] = w;
    if ((i & 3) == 0) sa[(size_t)m * (K >> 5) + (i >> 2)] = s;
}

hipError_t launch_quant_act_a4(uint32_t* aq, float* sa, const float* x, int rows, int K, hipStream_t st) {
    const dim3 grid((K / 8 + 255) / 256, rows);
    const int aligned = ((uintptr_t)x & 15) == 0;
    hipLaunchKernelGGL(quant_act_a4_k, grid, dim3(256), 0, st, x, aq, sa, K, aligned);
    return hipGetLastError();
}

// ---------------------------------------------------------------------------
// RT4 fp16 row-major weight scales -> fp32 group-major (src/model.cpp:190-202,
// a host loop in the reference).  One thread per output element; writes are
// coalesced, reads stride by NG.
__global__ __launch_bounds__(256) void make_group_major_k(const uint16_t* __restrict__ ws,
                                                          float* __restrict__ out, int N, int NG) {
    const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
    if (i >= (size_t)N * NG) return;
    const int g = (int)(i / N), n = (int)(i % N);
    out[i] = f16_bits_to_f32(ws[(size_t)n * NG + g]);
}

hipError_t launch_make_group_major(float* out, const uint16_t* ws, int N, int NG, hipStream_t st) {
    const size_t tot = (size_t)N * NG;
    hipLaunchKernelGGL(make_group_major_k, dim3((unsigned)((tot + 255) / 256)), dim3(256), 0, st, ws, out,
                       N, NG);
    return hipGetLastError();
}

}  // namespace rt4
