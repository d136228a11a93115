// A caller that keeps the reference's decode attention (src/k_fa.hip:244-259)
// in its own link, as src/model.cpp's build would: the library's k_attention
// must hand the single-row decode branch (n_row == 1, off + 1 == n_kv) to it.
// No device work happens: the stand-in decode routine only reports its call.
#include <cstdio>
#include <cstdlib>

#include "rt4_kernels.h"

void k_attention_decode(float*, const u32*, const float*, const u32*, const float*, const u32*, const float*,
                        int n_kv, int kv_cap, int n_heads, int ratio, int n_q, float*, float*, float*,
                        int max_split) {
    printf("decode n_kv=%d kv_cap=%d n_heads=%d ratio=%d n_q=%d max_split=%d\n", n_kv, kv_cap, n_heads, ratio, n_q,
           max_split);
    fflush(stdout);
    exit(7);
}

int main() {
    k_attention(nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, 64, 1, 300, 299, 5, 24, 6, 4096,
                nullptr, nullptr, nullptr, 8);
    return 0;  // not reached
}
