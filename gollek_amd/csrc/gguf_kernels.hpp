// gguf_kernels.hpp -- host-side launchers of the gfx950 kernels.  All
// launchers are asynchronous on `stream` and take device pointers; argument
// validation happens in the C-ABI layer (gguf_capi.hip).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gollek {

// Tunables read by the launchers.  Zero means "pick automatically".
struct LaunchTuning {
    int cu_count = 256;          // compute units of the current device
    int64_t gemv_rows_per_wave = 0;
    int gemv_row_batch = 0;      // rows per load batch (1, 2, 4, 8)
    int gemv_waves_per_cu = 8;   // target resident waves per CU
    int gemm_variant = 0;
    int gemv_variant = 0;        // 1 forces the fp32 GEMV kernels
};
LaunchTuning &tuning();

hipError_t launch_dequant(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                          int64_t row0, int64_t nrows, float *out, hipStream_t stream);

// y[r] = sum_k W[r, k] * x[k] for r < rows.
hipError_t launch_gemv(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                       const float *x, float *y, int64_t rows, hipStream_t stream);

// Q4_K GEMV with integer dot products (gguf_gemv_dot4.hip).
bool q4k_dot4_supported(int64_t row_bytes, int64_t cols, const void *w, const float *x);
hipError_t launch_gemv_q4k_dot4(const uint8_t *w, int64_t row_bytes, int64_t cols,
                                const float *x, float *y, int64_t rows, hipStream_t stream);

// Name of the GEMV kernel variant launch_gemv picks (for profiling notes).
const char *gemv_variant_name(int type_id, int64_t row_bytes, int64_t cols, const void *w,
                              const float *x);

}  // namespace gollek
