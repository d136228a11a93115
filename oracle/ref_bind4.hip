// ref_bind4.hip -- C-callable handle onto the reference's int4 decode activation
// quantizer (quant_act4, kernels/gemv_w4a4_core.h:22-44), compiled in place
// from /root/reference for gfx950 by oracle/Makefile into oracle/_ref/libref_hip.so.
//
// TEST INFRASTRUCTURE ONLY: used by tests/ as a third-party check of the CPU
// oracle and of our HIP quantizer on the same inputs.  Nothing in the product
// library links this.  Its own translation unit: the header shares macro names
// with gemv_w4a8_core.h.  The header's GEMV kernel (v_dot8_i32_i4 inline asm,
// gfx926 code) is a template that is never instantiated here, so it is not built.
#include "gemv_w4a4_core.h"  // resolved via -I<reference>/kernels

extern "C" {

// quant_act4, launched as src/k_gemv.hip:24-25 does: grid (K/32, rows) x 32
// threads; aq uint8 [rows][K/2], as f32 [rows][K/32] into caller device buffers.
void ref_quant_act4(const float* x, uint8_t* aq, float* as, int rows, int K) {
    quant_act4<<<dim3(K / SG, rows), 32>>>(x, aq, as, rows, K);
}

}  // extern "C"
