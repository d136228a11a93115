// rt4_dev.h -- device-side building blocks shared by the RT4 kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <hip/hip_fp16.h>
#include <cstdint>

namespace rt4 {

constexpr int kGroup = 128;       // RT4 quantization group along K (docs/FORMAT.md:61-73)
constexpr int kWave = 64;

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));
typedef float v32f __attribute__((ext_vector_type(32)));
typedef float v16f __attribute__((ext_vector_type(16)));

// fp16 bit pattern -> fp32 (exact).
__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
    return __half2float(__ushort_as_half(h));
}

// Wave-uniform value as an SGPR (lets loads indexed by it become scalar loads).
__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

// Max / sum across an aligned run of `W` lanes (W a power of two, <= 64).
template <int W>
__device__ __forceinline__ float run_max(float v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}
template <int W>
__device__ __forceinline__ int run_sum(int v) {
#pragma unroll
    for (int o = W / 2; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}

// int4 -> int8 unpack used by every MFMA kernel here.  An RT4 dword holds
// codes k=8d..8d+7 as nibbles, low nibble first, two's complement.  Shifting a
// nibble into the high half of a byte gives that byte the signed value 16*code
// exactly, so:
//   even(w): bytes = 16*code[8d+0,2,4,6]      odd(w): bytes = 16*code[8d+1,3,5,7]
// Every MFMA over these operands therefore returns 16x the integer dot product,
// which an arithmetic shift (or a 1/16 folded into an fp32 scale) removes
// exactly.  Activations are stored in the matching "interleaved" byte order:
// for each 8-element block, [a0 a2 a4 a6 | a1 a3 a5 a7].
__device__ __forceinline__ uint32_t even_x16(uint32_t w) { return (w << 4) & 0xF0F0F0F0u; }
__device__ __forceinline__ uint32_t odd_x16(uint32_t w) { return w & 0xF0F0F0F0u; }

// Saturating helpers for the quantizers (same clamp order as the reference).
__device__ __forceinline__ int clampi(int v, int lo, int hi) { return v > hi ? hi : (v < lo ? lo : v); }

// x / s rounded to nearest through the reciprocal: y = RN(1/s) (hipcc's division
// is correctly rounded), t = RN(x*y), then one correction RN(t + RN(x - t*s)*y)
// with both steps fused.  Markstein's theorem gives RN(x/s) when t is faithful,
// and t is not faithful everywhere (x/s just below a power of two can put it more
// than one ulp away), so the equality with the IEEE quotient is not proven here.
// It is checked on exact CPU emulations of this sequence at the inputs where it
// could fail -- quotients within 8 ulp of every half-integer of the code range and
// of powers of two, all-ones significands, the quantizers' own distributions, and
// such a non-faithful t (tests/test_recip_div.py) -- and on the GPU against the
// reference's quantizer kernels, which divide.  The quantizers take this path
// only when every scale of the wave lies in [2^-96, 2^100]; tiny or non-finite
// scales divide.
__device__ __forceinline__ bool recip_div_ok(float s) { return s >= 0x1p-96f && s <= 0x1p+100f; }
__device__ __forceinline__ float div_by_recip(float x, float s, float y) {
    const float t = x * y;
    return fmaf(fmaf(-t, s, x), y, t);
}

// Agent-coherent (sc1) 4-byte vector store / load of split-tile partials, each
// with its wait in the same asm statement: the store has reached the coherent
// level before the counter increment that publishes it, and the load's value is
// valid before use.  (A release fence would write back the whole L2 instead.)
__device__ __forceinline__ void store_dev(float* p, float v) {
    asm volatile("global_store_dword %0, %1, off sc1\n\ts_waitcnt vmcnt(0) expcnt(0)" ::"v"(p), "v"(v) : "memory");
}
__device__ __forceinline__ float load_dev(const float* p) {
    float v;
    asm volatile("global_load_dword %0, %1, off sc1\n\ts_waitcnt vmcnt(0)" : "=&v"(v) : "v"(p) : "memory");
    return v;
}

// LDS byte address of a pointer into shared memory (wave-uniform).
__device__ __forceinline__ uint32_t lds_addr(const unsigned char* l) {
    return (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(uintptr_t)(__attribute__((address_space(3))) void*)l);
}
// A wave-uniform pointer as a scalar register pair.
__device__ __forceinline__ const void* sptr(const void* p) {
    const uint64_t v = (uint64_t)(uintptr_t)p;
    const uint32_t lo = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)v);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(v >> 32));
    return reinterpret_cast<const void*>((uintptr_t)(((uint64_t)hi << 32) | lo));
}
// global -> LDS: lane i's 16 (4) bytes at gbase + voff land at m0 + 16*i (4*i),
// m0 = lbase + IMM.  The scalar base keeps the per-lane address a 32-bit offset.
// m0 is a reserved register: the compiler holds no value in it across instructions
// and sets it right before each instruction that reads it, so these writes need
// no clobber (declaring one is refused with a warning).
template <int IMM>
__device__ __forceinline__ void dma16(uint32_t voff, const void* gbase, uint32_t lbase) {
    asm volatile("s_add_u32 m0, %2, %3\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sptr(gbase)),
                 "s"((uint32_t)__builtin_amdgcn_readfirstlane((int)lbase)), "n"(IMM)
                 : "memory");
}
template <int IMM>
__device__ __forceinline__ void dma4(uint32_t voff, const void* gbase, uint32_t lbase) {
    asm volatile("s_add_u32 m0, %2, %3\n\tglobal_load_lds_dword %0, %1" ::"v"(voff), "s"(sptr(gbase)),
                 "s"((uint32_t)__builtin_amdgcn_readfirstlane((int)lbase)), "n"(IMM)
                 : "memory");
}
}  // namespace rt4
