// rt4_internal.h -- launchers shared between the kernel files and the C ABI.
// Every launcher assumes its arguments were validated by the caller (capi.hip)
// and returns the launch status.
#pragma once
#include <hip/hip_runtime.h>
#include <cstdint>

namespace rt4 {

// ---- quantizers (quant.hip)
hipError_t launch_quant_act_a8(int8_t* xq, float* sa, int32_t* asu, const float* x, int rows,
                               int K, hipStream_t st);
bool quant_group_supported(int G);
hipError_t launch_quant_rows_a8(uint32_t* qh, uint32_t* ql, float* sc, float* sc16, int8_t* xq,
                                const float* x, int rows, int K, int G, int in_stride, int in_off,
                                hipStream_t st);
hipError_t launch_quant_rows_a4(uint32_t* q, float* sc, const float* x, int rows, int K, int G,
                                int in_stride, int in_off, hipStream_t st);
hipError_t launch_hl_to_i8(int8_t* xq, const uint32_t* qh, const uint32_t* ql, int rows, int K,
                           hipStream_t st);
hipError_t launch_make_group_major(float* out, const uint16_t* ws, int N, int NG, hipStream_t st);

// ---- decode GEMV (gemv.hip)
struct GemvCfg {
    int rt;     // 16-row weight tiles per workgroup (1 or 2)
    int waves;  // waves per workgroup; they split the K groups of the tile
};
constexpr int kGemvMaxGroupsPerWave = 10;  // weight loads one wave keeps in flight
constexpr int kGemvMaxWaves = 16;
constexpr size_t kGemvMaxActBytes = 160 * 1024;  // rows*K int8 staged in one workgroup's LDS
GemvCfg gemv_default_cfg(int rows, int N, int K);
bool gemv_cfg_valid(const GemvCfg& c, int K);
hipError_t launch_gemv_w4a8(float* y, int32_t* gsum, const uint32_t* wq, const uint16_t* ws,
                            const int8_t* xq, const float* sa, int rows, int N, int K,
                            const GemvCfg& cfg, hipStream_t st);

}  // namespace rt4
