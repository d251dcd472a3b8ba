// gguf_kernels.hpp -- host-side launchers of the gfx950 kernels.  All
// launchers are asynchronous on `stream` and take device pointers; argument
// validation happens in the C-ABI layer (gguf_capi.hip).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <stdint.h>

namespace gollek {

// Kernel selection read by the launchers (gollek_hip_testing_set_option).
// Process-wide and atomic: a set_option call on one thread and launches on
// others do not race, and a launch sees either the old or the new value.
// Zero means "pick automatically".
struct LaunchTuning {
    std::atomic<int> cu_count{256};          // compute units of the current device
    std::atomic<int> gemv_variant{0};        // 0 auto (matrix cores), 1 fp32 kernels,
                                             // 3 Q4_K on shared tiles for K <= 4096, 4 Q8_0 / Q4_0
                                             // rings and Q5_K / Q6_K fp32
    std::atomic<int> moe_variant{0};         // 0 auto (matrix cores), 1 v_dot4 expert kernels
};
LaunchTuning &tuning();

// Compute units of the current device (256 until a device is initialised).
inline int device_cus() {
    const int c = tuning().cu_count.load(std::memory_order_relaxed);
    return c > 0 ? c : 256;
}

hipError_t launch_dequant(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                          int64_t row0, int64_t nrows, float *out, hipStream_t stream);

// y[r] = sum_k W[r, k] * x[k] for r < rows.  prep: the matrix's prepared
// column layout for prep_rows rows per workgroup (launch_prepare_col_layout),
// used when the column kernel takes the shape with that partition.
hipError_t launch_gemv(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                       const float *x, float *y, int64_t rows, hipStream_t stream,
                       const uint8_t *prep = nullptr, int64_t prep_rows = 0);

// The column kernel's partition of a full mat-vec (rows per workgroup; 0
// when the column kernel does not take the shape) and the prepared layout
// for it: every workgroup's block of rows stored superblock column by
// column (same bytes; gguf_gemv_mfma.hip).
int64_t col_layout_rows(int type_id, int64_t rows, int64_t cols);
hipError_t launch_prepare_col_layout(int type_id, const uint8_t *raw, uint8_t *prep, int64_t rows,
                                     int64_t row_bytes, int64_t per, hipStream_t stream);
// A full mat-vec read from the prepared layout only (hipErrorInvalidValue
// when the partition is no longer prep_rows or x is not 16-byte aligned).
hipError_t launch_gemv_prepared(int type_id, const uint8_t *prep, int64_t row_bytes, int64_t cols, const float *x,
                                float *y, int64_t rows, int64_t prep_rows, hipStream_t stream);
// The inverse for rows row0 .. row0 + nrows - 1 of the prepared layout:
// their GGUF bytes, packed (nrows x row_bytes) into dst.
hipError_t launch_gather_col_rows(int type_id, const uint8_t *prep, uint8_t *dst, int64_t rows, int64_t row_bytes,
                                  int64_t per, int64_t row0, int64_t nrows, hipStream_t stream);

// Q4_K GEMV on the matrix cores (gguf_gemv_mfma.hip).
// Q8_0 / Q4_0 GEMV through per-wave buffer->LDS rings (gguf_gemv_ring.hip).
bool gemv_ring_supported(int type_id, int64_t row_bytes, int64_t cols, int64_t rows, const void *w,
                         const float *x);
hipError_t launch_gemv_ring(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                            const float *x, float *y, int64_t rows, hipStream_t stream);
bool q4k_mfma_supported(int64_t row_bytes, int64_t cols, int64_t rows, const void *w,
                        const float *x);
hipError_t launch_gemv_q4k_mfma(const uint8_t *w, int64_t row_bytes, int64_t cols,
                                const float *x, float *y, int64_t rows, hipStream_t stream,
                                const uint8_t *prep = nullptr, int64_t prep_rows = 0);
// Q4_0 / Q8_0 / Q5_K on the matrix cores (gguf_gemv_mfma.hip, the column
// kernel): K a multiple of 256 up to 4096, any row count.
bool q32_mfma_supported(int type_id, int64_t row_bytes, int64_t cols, int64_t rows, const void *w,
                        const float *x);
hipError_t launch_gemv_q32_mfma(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                                const float *x, float *y, int64_t rows, hipStream_t stream,
                                const uint8_t *prep = nullptr, int64_t prep_rows = 0);

// Q6_K on the matrix cores (gguf_gemv_q6k_mfma.hip): K a multiple of 2048 up
// to 14336, row bytes K / 256 * 210, weights and x 16-byte aligned.
// Q5_K past K = 4096 on the matrix cores (gguf_gemv_mfma.hip, the K > 4096
// Q4_K kernel with the fifth bit): K a multiple of 256 up to 16384.
bool q5k_wide_mfma_supported(int64_t row_bytes, int64_t cols, int64_t rows, const void *w, const float *x);
hipError_t launch_gemv_q5k_wide_mfma(const uint8_t *w, int64_t row_bytes, int64_t cols, const float *x, float *y,
                                     int64_t rows, hipStream_t stream);
bool q6k_mfma_supported(int64_t row_bytes, int64_t cols, int64_t rows, const void *w, const float *x);
hipError_t launch_gemv_q6k_mfma(const uint8_t *w, int64_t row_bytes, int64_t cols, const float *x, float *y,
                                int64_t rows, hipStream_t stream);

// Q5_K / Q6_K (gguf_k56.hip): dequantization and the GEMV; the GEMV needs
// gemv_k56_supported (x 16-byte aligned, Q6_K weights 2-byte and Q5_K
// weights 4-byte aligned); launch_gemv runs other buffers on the generic
// kernel.
bool is_k56(int type_id);
hipError_t launch_dequant_k56(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                              int64_t row0, int64_t nrows, float *out, hipStream_t stream);
bool gemv_k56_supported(int type_id, int64_t row_bytes, const void *w, const float *x);
hipError_t launch_gemv_k56(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                           const float *x, float *y, int64_t rows, hipStream_t stream);


// Y[M, N] = X[M, K] (bf16 bits) . W[N, K]^T for Q8_0, Q4_0 or Q4_K W
// (gguf_gemm.hip, gguf_gemm_tile.hip).  Shapes whose output tiles leave CUs
// idle are split over K into partial tiles in `workspace` (device memory of
// gemm_workspace_bytes(type, M, N, K) bytes; with less they split less or
// run unsplit) and added in split order.
size_t gemm_workspace_bytes(int type_id, int M, int N, int K);
// The largest gemm_workspace_bytes(type, M, N, K) over every M.
size_t gemm_workspace_max_bytes(int type_id, int N, int K);
// prep / prep_rows: the weight's prepared column layout (M <= 4 reads it
// when its partition is the column kernel's; w may then be nullptr, a
// compacted handle, and the call fails for shapes that need the GGUF rows).
hipError_t launch_gemm_bf16(int type_id, const uint8_t *w, int64_t row_bytes, const uint16_t *x, float *y,
                            int M, int N, int K, hipStream_t stream, float *workspace = nullptr,
                            size_t workspace_bytes = 0, const uint8_t *prep = nullptr, int64_t prep_rows = 0);
// M = 1 .. 4 on the GEMV's column kernel (gguf_gemv_mfma.hip): two vectors
// in each MFMA over one stream of the weights.
bool gemm_col_supported(int type_id, int64_t row_bytes, int M, int N, int K, const void *w, const void *x);
hipError_t launch_gemm_col(int type_id, const uint8_t *w, int64_t row_bytes, const uint16_t *x, float *y, int M,
                           int N, int K, hipStream_t stream, const uint8_t *prep = nullptr,
                           int64_t prep_rows = 0);
// The 128 x 128 tile kernel (gguf_gemm_tile.hip).
bool gemm_tile_supported(int type_id, int64_t row_bytes, int M, int N, int K, const void *w,
                         const void *x, const void *y);
size_t gemm_tile_workspace_bytes(int type_id, int M, int N, int K);
hipError_t launch_gemm_tile(int type_id, const uint8_t *w, int64_t row_bytes, const uint16_t *x,
                            float *y, int M, int N, int K, hipStream_t stream, float *workspace,
                            size_t workspace_bytes);

// Workspace layout of the grouped MoE FFN (byte offsets; gguf_moe.hip).
struct MoeLayout {
    size_t meta, xdig, xdig_stride, h, hdig, hdig_stride, ypair, total;
    int64_t meta_ints;
};
MoeLayout moe_layout(int64_t tokens, int64_t top_k, int64_t hidden, int64_t inter, int64_t experts);

// out[T, H] = sum_j w[t,j] down_e(silu(gate_e x_t) * up_e x_t) for stacked
// gate / up / down experts of types Q8_0, Q4_0, Q4_K, Q5_K or Q6_K (each
// matrix its own type): the matrix-core passes for Q4_K, Q5_K or Q6_K gate /
// up (moe_kq_mfma_supported) and for all-Q4_0 where they take the shape, the
// v_dot4 passes for all-Q4_K otherwise, the row kernels for everything else;
// ws must hold moe_layout(...).total bytes.
hipError_t launch_moe(int gate_type, int up_type, int down_type, const uint8_t *gate, const uint8_t *up,
                      const uint8_t *down, int64_t gate_row_bytes, int64_t up_row_bytes,
                      int64_t down_row_bytes, int E, int H, int I, const float *x, const int32_t *ids,
                      const float *wts, int T, int top_k, float *out, uint8_t *ws, hipStream_t stream);
// The shared expert (gguf_moe.hip): out[t] += g_t * ffn(x_t) over one
// expert of `inter` rows, g_t from the gate_inp row (nullptr: 1); ws holds
// moe_shared_layout(...).total bytes (y, the routes, the FFN's workspace).
struct MoeSharedLayout {
    size_t y, ids, wts, ffn, total;
};
MoeSharedLayout moe_shared_layout(int64_t tokens, int64_t hidden, int64_t inter);
hipError_t launch_moe_shared(int gate_type, int up_type, int down_type, const uint8_t *gate, const uint8_t *up,
                             const uint8_t *down, int64_t gate_row_bytes, int64_t up_row_bytes,
                             int64_t down_row_bytes, int H, int I, const float *x, const float *gate_inp, int T,
                             float *out, uint8_t *ws, hipStream_t stream);
hipError_t launch_moe_q4k_dot4(const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                               int64_t gate_row_bytes, int64_t down_row_bytes, int E, int H, int I,
                               const float *x, const int32_t *ids, const float *wts, int T, int top_k,
                               float *out, uint8_t *ws, hipStream_t stream);
// Routes (tokens x top_k) one launch of the matrix-core passes routes in LDS.
constexpr int kMoeMfmaMaxRoutes = 2048;
// K-quant experts on the matrix-core passes (gguf_moe_mfma.hip): gate / up
// both Q4_K or both Q5_K (hidden up to 4096) or both Q6_K (hidden up to 2048,
// an even number of superblocks); down rows
// Q4_K, Q5_K or Q6_K through the token-major pass (inter up to 1024), else
// Q4_K or Q5_K through the expert-major pass; hidden and inter multiples of
// 256, x 16-byte aligned.
bool moe_kq_mfma_supported(int gate_type, int down_type, int E, int H, int I, int T, int top_k,
                           const float *x);
hipError_t launch_moe_kq_mfma(int gate_type, int down_type, const uint8_t *gate, const uint8_t *up,
                              const uint8_t *down, int E, int H, int I, const float *x, const int32_t *ids,
                              const float *wts, int T, int top_k, float *out, uint8_t *ws, hipStream_t stream);
// All-Q4_0 experts on the matrix-core passes (hidden up to 2048, hidden and
// inter multiples of 256; x 16-byte aligned).
bool moe_q40_mfma_supported(int E, int H, int I, int P, const float *x);
hipError_t launch_moe_q40_mfma(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int E, int H, int I,
                               const float *x, const int32_t *ids, const float *wts, int T, int top_k, float *out,
                               uint8_t *ws, hipStream_t stream);

// Pieces of the MoE pipeline shared by its two implementations (gguf_moe.hip,
// gguf_moe_mfma.hip): routing (meta layout of moe_layout; tiles0 / tiles1 =
// work items per expert and route group of the matrix-core passes) and the
// route-order combine.
hipError_t launch_moe_route(const int32_t *ids, const float *wts, int P, int E, int tiles0,
                            int tiles1, int32_t *meta, hipStream_t stream);
hipError_t launch_moe_combine(const int32_t *ids, const float *wts, const float *ypair, int T,
                              int top_k, int H, int E, float *out, hipStream_t stream);
// MoE router (gguf_moe_router.hip): logits [T, E] -> ids / wts [T, K] with
// softmax (sigmoid = 0) or sigmoid scoring and renormalised top-K weights.
size_t moe_topk_lds_bytes(int E, int K);
hipError_t launch_moe_topk(const float *logits, int T, int E, int K, int sigmoid, int32_t *ids,
                           float *wts, hipStream_t stream);

}  // namespace gollek

// Pieces of the C ABI (gguf_capi.hip) the GGUF file loader (gguf_file.hip) uses.
struct gollek_hip_weight;
namespace gollek {

// Sets what gollek_hip_last_status / gollek_hip_last_error report.
void record_status(int32_t code, const char *message);
// A weight handle on the current device that owns an uninitialised
// rows * row_bytes device buffer; same validation and messages as
// gollek_hip_weight_upload.  nullptr (with the error recorded) on failure.
gollek_hip_weight *weight_alloc_owned(int32_t type_id, int64_t rows, int64_t cols, int64_t row_bytes,
                                      char *err, size_t err_len);
uint8_t *weight_data(gollek_hip_weight *w);

// Name of the GEMV kernel variant launch_gemv picks (for profiling notes).
const char *gemv_variant_name(int type_id, int64_t row_bytes, int64_t cols, const void *w,
                              const float *x);

}  // namespace gollek
