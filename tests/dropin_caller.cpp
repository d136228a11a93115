// dropin_caller.cpp -- a stand-in for the reference runtime's use of the RT4 path,
// written against include/rt4_kernels.h and librt4k.so only (plus the HIP runtime
// for device memory and copies, as the reference's runtime uses it).
//
// It repeats the call sequences of src/model.cpp:
//   linear_quant (src/model.cpp:1010-1026): M <= 4 -> k_gemv_w4a8; otherwise M is
//     padded to a multiple of 128, k_quant_rows_a8 (default in_stride / in_off),
//     then k_gemm_i4_a8 with its c2 scratch;
//   the attention prefill (src/model.cpp:1077-1081, :1140): k_attn_q_quant over the
//     T new rows (scales laid out for TP rows), k_kv_append_k / k_kv_append_v at
//     seq_len, then k_attention with n_q = TP, n_row = T.
// Inputs and outputs are raw little-endian files in the directory given as argv[1]
// (names below); the shapes come from argv.  Used by tests/test_gpu_dropin.py.
//
//   dropin_caller DIR gemv M N K        x.f32 [M][K], wq.u32 [N][K/8], ws.u16 [N][K/128] -> y.f32 [M][N]
//   dropin_caller DIR gemm M N K        x.f32 [Mp][K] (rows >= M: padding), wq, wsgm.f32 [K/128][N]
//                                       -> c.f32 [Mp][N]
//   dropin_caller DIR attn T H KVH seq_len cap
//                                       q.f32 [T][H][256], kold/vold.f32 [seq_len][KVH][256],
//                                       knew/vnew.f32 [T][KVH][256] -> out.f32 [H][TP][256] and the
//                                       quantized qq, qs, kc, ksc, vc, vsc
#include <hip/hip_runtime.h>

#include <cstdio>
#include <cstdlib>
#include <string>
#include <vector>

#include "rt4_kernels.h"

namespace {

std::string g_dir;

void check(hipError_t e, const char* what) {
    if (e != hipSuccess) {
        std::printf("%s: %s\n", what, hipGetErrorString(e));
        std::exit(3);
    }
}

std::vector<char> read_file(const char* name, size_t bytes) {
    std::vector<char> v(bytes);
    FILE* f = std::fopen((g_dir + "/" + name).c_str(), "rb");
    if (!f || std::fread(v.data(), 1, bytes, f) != bytes) {
        std::printf("cannot read %zu bytes of %s\n", bytes, name);
        std::exit(4);
    }
    std::fclose(f);
    return v;
}

template <typename T>
T* upload(const char* name, size_t count) {
    const std::vector<char> h = read_file(name, count * sizeof(T));
    void* d = nullptr;
    check(hipMalloc(&d, count * sizeof(T)), "hipMalloc");
    check(hipMemcpy(d, h.data(), count * sizeof(T), hipMemcpyHostToDevice), "hipMemcpy H2D");
    return static_cast<T*>(d);
}

template <typename T>
T* device(size_t count) {
    void* d = nullptr;
    check(hipMalloc(&d, count * sizeof(T)), "hipMalloc");
    check(hipMemset(d, 0, count * sizeof(T)), "hipMemset");
    return static_cast<T*>(d);
}

float* ones(size_t count) {
    float* d = device<float>(count);
    const std::vector<float> h(count, 1.f);
    check(hipMemcpy(d, h.data(), count * sizeof(float), hipMemcpyHostToDevice), "hipMemcpy ones");
    return d;
}

template <typename T>
void download(const char* name, const T* d, size_t count) {
    std::vector<T> h(count);
    check(hipMemcpy(h.data(), d, count * sizeof(T), hipMemcpyDeviceToHost), "hipMemcpy D2H");
    FILE* f = std::fopen((g_dir + "/" + name).c_str(), "wb");
    if (!f || std::fwrite(h.data(), sizeof(T), count, f) != count) {
        std::printf("cannot write %s\n", name);
        std::exit(5);
    }
    std::fclose(f);
}

// Model::linear_quant without the RT_ACT4 branch (src/model.cpp:1010-1026)
void linear_quant(float* y, const u32* wq, const float* ws, const float* wsgm, const float* x, int M, int N, int K,
                  u32* aq_h, u32* aq_l, float* asc8, float* asc16, float* c_tmp) {
    if (M <= 4) {
        k_gemv_w4a8(y, wq, ws, x, M, N, K);
    } else {
        const int Mp = (M + 127) / 128 * 128;
        k_quant_rows_a8(aq_h, aq_l, asc8, asc16, x, Mp, K, 128);
        k_gemm_i4_a8(y, c_tmp, wq, wsgm, aq_h, aq_l, asc8, asc16, Mp, N, K);
    }
}

}  // namespace

int main(int argc, char** argv) {
    if (argc < 3) {
        std::printf("usage: dropin_caller DIR gemv|gemm|attn ...\n");
        return 2;
    }
    g_dir = argv[1];
    const std::string what = argv[2];
    if ((what == "gemv" || what == "gemm") && argc == 6) {
        const int M = std::atoi(argv[3]), N = std::atoi(argv[4]), K = std::atoi(argv[5]);
        const int Mp = what == "gemm" ? (M + 127) / 128 * 128 : M;
        u32* wq = upload<u32>("wq.u32", (size_t)N * K / 8);
        float* x = upload<float>("x.f32", (size_t)Mp * K);
        float* ws = nullptr;
        float* wsgm = nullptr;
        if (what == "gemv")
            ws = reinterpret_cast<float*>(upload<uint16_t>("ws.u16", (size_t)N * K / 128));
        else
            wsgm = upload<float>("wsgm.f32", (size_t)K / 128 * N);
        // the runtime's activation scratch (sized for this call)
        u32* aq_h = device<u32>((size_t)Mp * K / 8);
        u32* aq_l = device<u32>((size_t)Mp * K / 8);
        float* asc8 = device<float>((size_t)Mp * K / 128);
        float* asc16 = device<float>((size_t)Mp * K / 128);
        float* c_tmp = device<float>((size_t)Mp * N);
        float* y = device<float>((size_t)Mp * N);
        linear_quant(y, wq, ws, wsgm, x, M, N, K, aq_h, aq_l, asc8, asc16, c_tmp);
        check(hipDeviceSynchronize(), "linear_quant");
        download(what == "gemv" ? "y.f32" : "c.f32", y, (size_t)Mp * N);
        std::printf("%s ok M=%d N=%d K=%d\n", what.c_str(), M, N, K);
        return 0;
    }
    if (what == "attn" && argc == 8) {
        const int T = std::atoi(argv[3]), H = std::atoi(argv[4]), KV = std::atoi(argv[5]);
        const int seq_len = std::atoi(argv[6]), cap = std::atoi(argv[7]);
        const int D = 256, BG = 64, TP = (T + 63) / 64 * 64, n_kv = seq_len + T;
        float* q = upload<float>("q.f32", (size_t)T * H * D);
        float* kold = upload<float>("kold.f32", (size_t)seq_len * KV * D);
        float* vold = upload<float>("vold.f32", (size_t)seq_len * KV * D);
        float* knew = upload<float>("knew.f32", (size_t)T * KV * D);
        float* vnew = upload<float>("vnew.f32", (size_t)T * KV * D);
        // as Model::reset_state leaves them (src/model.cpp:982-1000): zero codes, unit scales
        u32* qq = device<u32>((size_t)H * TP * (D / 8));
        float* qs = ones((size_t)H * 2 * TP);
        u32* kc = device<u32>((size_t)KV * cap * (D / 8));
        float* ksc = ones((size_t)KV * 2 * cap);
        u32* vc = device<u32>((size_t)KV * (cap / 8) * D);
        float* vsc = ones((size_t)KV * (cap / BG) * D);
        float* vstage = device<float>((size_t)KV * BG * D);
        float* out = device<float>((size_t)H * TP * D);
        float* pout = device<float>((size_t)4 * 24 * 8 * 256);
        float* pmax = device<float>((size_t)4 * 24 * 8);
        float* psum = device<float>((size_t)4 * 24 * 8);
        // the cache as an earlier prefill chunk left it, then this chunk
        if (seq_len > 0) {
            k_kv_append_k(kc, ksc, kold, 0, seq_len, KV, D, 128, cap);
            k_kv_append_v(vc, vsc, vstage, vold, 0, seq_len, KV, D, BG, cap);
        }
        k_attn_q_quant(qq, qs, q, T, H, D, 128, TP);
        k_kv_append_k(kc, ksc, knew, seq_len, T, KV, D, 128, cap);
        k_kv_append_v(vc, vsc, vstage, vnew, seq_len, T, KV, D, BG, cap);
        k_attention(out, qq, qs, kc, ksc, vc, vsc, TP, T, n_kv, seq_len, (n_kv + BG - 1) / BG, H, H / KV, cap,
                    pout, pmax, psum, 8);
        check(hipDeviceSynchronize(), "attention");
        download("out.f32", out, (size_t)H * TP * D);
        download("qq.u32", qq, (size_t)H * TP * (D / 8));
        download("qs.f32", qs, (size_t)H * 2 * TP);
        download("kc.u32", kc, (size_t)KV * cap * (D / 8));
        download("ksc.f32", ksc, (size_t)KV * 2 * cap);
        download("vc.u32", vc, (size_t)KV * (cap / 8) * D);
        download("vsc.f32", vsc, (size_t)KV * (cap / BG) * D);
        std::printf("attn ok T=%d H=%d KV=%d seq_len=%d cap=%d\n", T, H, KV, seq_len, cap);
        return 0;
    }
    std::printf("bad arguments\n");
    return 2;
}
