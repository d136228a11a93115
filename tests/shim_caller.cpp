// A caller of the reference-compatible API, as src/model.cpp would be: it
// includes the prototypes, links librt4k.so, and calls k_gemv_w4a8 with a shape
// the reference rejects (rows > 4), which must print and exit(1) before any
// device work.
#include "rt4_kernels.h"

int main() {
    static float y[8], x[8];
    static u32 wq[8];
    static float ws[8];
    k_gemv_w4a8(y, wq, ws, x, 5, 64, 256);
    return 0;  // not reached
}
