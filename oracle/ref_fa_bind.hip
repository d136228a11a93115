// ref_fa_bind.hip -- a C-callable handle onto the reference's int4 FlashAttention
// prefill kernel (fa_int4, kernels/flash_attn_core.h:74-435), compiled in place
// from /root/reference for gfx950 by oracle/Makefile into oracle/_ref/libref_hip.so.
//
// TEST INFRASTRUCTURE ONLY: tests/test_attention.py runs it on the same seeded
// quantized caches as our kernel (test_attention_against_reference_kernel, and the
// full configs[4] shape).  Its integer dot products are `v_dot8_i32_i4` inline
// assembly (flash_attn_core.h:61-64), which gfx950 implements with the same signed
// int4 semantics; the tests first check this build against the CPU algorithm model
// (rt4o_fa_rows mode 1) and then our kernel against this build.
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
