// rt4_internal.h -- launchers shared between the kernel files and the C ABI.
// Every launcher assumes its arguments were validated by the caller (capi.hip)
// and returns the launch status.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace rt4 {

// Records msg as this thread's rt4_last_error() text and returns code.
int set_error(int code, const char* msg);

// ---- quantizers (quant.hip)
hipError_t launch_quant_act_a8(int8_t* xq, float* sa, int32_t* asu, const float* x, int rows,
                               int K, hipStream_t st);
bool quant_group_supported(int G);
hipError_t launch_quant_row(int8_t* xq, float* sa, int32_t* asu, const float* x, int rows, int K, int mode,
                            hipStream_t st);
hipError_t launch_quant_rows_a8(uint32_t* qh, uint32_t* ql, float* sc, float* sc16, int8_t* xq,
                                const float* x, int rows, int K, int G, int in_stride, int in_off,
                                hipStream_t st);
hipError_t launch_quant_rows_a4(uint32_t* q, float* sc, const float* x, int rows, int K, int G,
                                int in_stride, int in_off, hipStream_t st);
// q8 = 16h + l from digit planes, or the sign-extended l alone when qh is null.
hipError_t launch_hl_to_i8(int8_t* xq, const uint32_t* qh, const uint32_t* ql, int rows, int K,
                           hipStream_t st);
hipError_t launch_quant_act_a4(uint32_t* aq, float* sa, const float* x, int rows, int K, hipStream_t st);
hipError_t launch_make_group_major(float* out, const uint16_t* ws, int N, int NG, hipStream_t st);

// ---- decode GEMV (gemv.hip)
struct GemvCfg {
    int gpw;    // K groups per wave (even, 2..12)
    int waves;  // waves per workgroup; they share one tile and split its K groups
    int max_split;  // leftover tiles are cut along K into at most this many pieces (1: never,
                    // 0: as many as keep 32 groups per piece)
    int rb;     // 16-row blocks per tile (1 or 2): a wave applies its activations to rb blocks
    int dot = 0;  // one activation row, pre-quantized: the row-contiguous dot-product form with
                  // this many weight rows per wave (1 or 2); 0: the MFMA forms above
};
constexpr int kGemvMaxWaves = 16;
constexpr int kGemvDotWaves = 2;       // waves per workgroup of the dot-product form
constexpr int kGemvMaxSplit = 64;      // largest k_splits override
constexpr int kGemvMaxRb = 2;
constexpr int kGemvRb2MinRows = 3;     // default rb = 2 needs this many activation rows
constexpr int kGemvRb2Work = 320;      // and this many (32-row tile x K group) units per CU
GemvCfg gemv_default_cfg(int rows, int N, int K, int cus);
GemvCfg gemv_mfma_cfg(int rows, int N, int K, int cus);   // the default among the MFMA forms
bool gemv_cfg_valid(const GemvCfg& c, int K);
// Grid of the GEMV: `full` whole tiles of 16*rb rows, then `nrem` tiles cut along
// K into S pieces each, whose partials (part: nrem*S*rb*rows*16 floats) are summed
// by the last piece to arrive (cnt: nrem counters, zero between calls).
struct GemvSplit {
    int full, nrem, S;
    float* part;
    int* cnt;
};
GemvSplit gemv_split(int N, int K, const GemvCfg& c, int cus);
size_t gemv_part_bytes(const GemvSplit& sp, int rows, int rb);
// Activations either pre-quantized (xq, sa; xf null) or fp32 xf [rows][K], 16-byte
// aligned, quantized inside the kernel exactly as launch_quant_act_a8 would.
hipError_t launch_gemv_w4a8(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws,
                            const int8_t* xq, const float* sa, const float* xf, int rows, int N, int K,
                            const GemvCfg& cfg, const GemvSplit& sp, hipStream_t st);

// ---- W4A4 decode GEMV (gemv4.hip): y f32 [rows][N] from RT4 weights and int4
// activation codes aq u32 [rows][K/8] with scales sa f32 [rows][K/32].  Tiles of
// 16 rows (rb 1), gpw 2 or 4, waves capped at the chunk count; leftover tiles cut
// along K as gemv_split plans (partials nrem*S*rows*16 floats).
GemvCfg gemv4_default_cfg(int rows, int N, int K, int cus);
bool gemv4_cfg_valid(const GemvCfg& c);
hipError_t launch_gemv_w4a4(float* y, const uint32_t* wq, const uint16_t* ws, const uint32_t* aq, const float* sa,
                            int rows, int N, int K, const GemvCfg& c, const GemvSplit& sp, hipStream_t st);

// ---- prefill GEMM (gemm.hip)
// C f32 [M][N] from int8 codes A [M][K] (interleaved), RT4 weights W [N][K/8],
// group-major scales sa [K/128][M] and sb [K/128][N]; gsum (optional, tests)
// receives the exact per-group int32 dot products [M][N][K/128].  The launch is
// persistent (one workgroup per CU, equal shares of the (tile, group) units);
// `part` and `cnt` are its split-tile workspace: part_bytes of partial sums and
// cnt_bytes of counters that must be zero before the first launch (every launch
// leaves them zero again).
struct GemmPlan {
    int ntm, ntn, ntiles, P;
    long long T;
    size_t part_bytes, cnt_bytes;
};
GemmPlan gemm_plan(int M, int N, int K, int cus);
hipError_t launch_gemm_w4a8(float* C, int32_t* gsum, const int8_t* A, const uint32_t* W,
                            const float* sa, const float* sb, int M, int N, int K, const GemmPlan& plan,
                            float* part, int* cnt, hipStream_t st);
hipError_t launch_zero_i32(int* p, size_t n, hipStream_t st);

// ---- int4-KV attention (attn.hip); head dim 256, Q/K groups of 128, V tiles of 64 keys
hipError_t launch_attn_q_quant(uint32_t* qq, float* qs, const float* x, int T, int H, int D, int G, int TP,
                               hipStream_t st);
hipError_t launch_kv_append_k(uint32_t* kc, float* ksc, const float* kf, int t0, int T, int H, int D, int G,
                              int kv_total, hipStream_t st);
hipError_t launch_kv_append_v(uint32_t* vc, float* vsc, float* stage, const float* vf, int t0, int T, int H,
                              int D, int BG, int kv_total, hipStream_t st);
// KV splits per (query block, head) that balance the grid over `cus` CUs, and
// the workspace they need (0 for one split): partial states, and one counter per
// (query block, head) that must be zero before the first launch (every launch
// leaves them zero again).
int fa_splits(int n_q, int n_heads, int n_tile, int cus);
size_t fa_part_bytes(int n_q, int n_heads, int nsplit);
size_t fa_cnt_bytes(int n_q, int n_heads, int nsplit);
// Bytes of the staged K/V copy the DMA form of the prefill reads (two 16 KB blocks
// per tile and KV head).  launch_fa_int4 with kvx (that many bytes) fills it and runs
// the DMA form; with kvx null each workgroup stages its tiles itself.  Same results.
size_t fa_kvx_bytes(int n_heads, int ratio, int n_tile);
hipError_t launch_fa_int4(float* out, const uint32_t* qq, const float* qsc, const uint32_t* kc, const float* ksc,
                          const uint32_t* vc, const float* vsc, int n_q, int n_kv, int off, int n_tile,
                          int n_heads, int ratio, int kv_cap, int nsplit, float* part, int* cnt, void* kvx,
                          hipStream_t st);

}  // namespace rt4
