// ref_fa_bind.hip -- a C-callable handle onto the reference's int4 FlashAttention
// prefill kernel (fa_int4, kernels/flash_attn_core.h:74-435), compiled in place
// from /root/reference for gfx950 by oracle/Makefile into oracle/_ref/libref_hip.so.
//
// TEST INFRASTRUCTURE ONLY: tests/ run it on the same seeded inputs as a
// third-party check of the CPU oracle's algorithm model and of our kernel.  Its
// integer dot products are `v_dot8_i32_i4` inline assembly (flash_attn_core.h:61-64),
// which gfx950 also implements; whether the gfx950 build computes the
// reference's results is itself checked against the CPU oracle by the test
// before the build is used as a reference.
#include <hip/hip_runtime.h>
#include <cstdint>
typedef uint32_t u32;
#include "flash_attn_core.h"  // resolved via -I<reference>/kernels

extern "C" void ref_fa_int4(const u32* Q, const float* Qs, const u32* K, const float* Ks, const u32* V,
                            const float* Vs, float* out, int n_q, int n_kv, int off, int n_tile,
                            int n_heads, int ratio, int kv_cap) {
    // launch shape of k_attention's prefill branch, src/k_fa.hip:294-296
    fa_int4<<<dim3((n_q + BM - 1) / BM, n_heads), NT>>>(Q, Qs, K, Ks, V, Vs, out, n_q, n_kv, off, n_tile,
                                                        ratio, kv_cap);
}
