/*
 * gollek_hip.h -- C ABI of the MI355X (gfx950) GGUF quantized linear-layer
 * library, libgollek_hip.so.
 *
 * The library is the native side of a drop-in for gollek's Java GGUF tensor
 * runtime (RT/ = runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/
 * gguf/runtime/).  The Java facade RT/GgufTensorOps keeps its signatures; an
 * FFM (java.lang.foreign) binding calls these functions from inside
 * RT/GgufMatVec.rows (RT/GgufMatVec.java:55-96) for ggml type ids 2 (Q4_0),
 * 8 (Q8_0), 12 (Q4_K), 13 (Q5_K) and 14 (Q6_K), ahead of the prepared and raw
 * Java routes.
 *
 * Conventions (those of the reference's own native bridge,
 * runner/gguf/gguf-fast-bridge/gollek_gguf_fast.cpp:672-800):
 *   - plain C types only: pointers, int32/int64 sizes, floats;
 *   - functions returning int return GOLLEK_HIP_OK (0) or a negative code;
 *     handle constructors return NULL on failure;
 *   - a message is written to the caller's `err` buffer (NUL-terminated,
 *     truncated to err_len) when err != NULL and err_len > 0;
 *   - the Java adapter maps codes back to the reference's exceptions:
 *     NULL -> NullPointerException (RT/GgufMatVec.java:32-35),
 *     ARG -> IllegalArgumentException (RT/GgufMatVec.java:65-71, :196-200;
 *            RT/GgufTensorOps.java:652-656; GC/core/GgmlType.java:70-81),
 *     UNSUPPORTED -> UnsupportedOperationException (RT/GgufRowDot.java:77-82,
 *            RT/GgufRowDequantizer.java:275),
 *     DEVICE / NOMEM -> IllegalStateException (no reference counterpart: the
 *            Java path has no device).
 *
 * Threading: every function may be called from any thread.  A weight handle
 * serialises its host-buffer calls with its own mutex (as the reference
 * bridge does per handle, gollek_gguf_fast.cpp:42) and runs them on its own
 * HIP stream; they return only when the output is in host memory.  The
 * *_device functions are asynchronous on the caller's stream and take device
 * pointers.
 */
#ifndef GOLLEK_HIP_H
#define GOLLEK_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define GOLLEK_HIP_OK 0
#define GOLLEK_HIP_ERR_NULL (-1)
#define GOLLEK_HIP_ERR_ARG (-2)
#define GOLLEK_HIP_ERR_UNSUPPORTED (-3)
#define GOLLEK_HIP_ERR_DEVICE (-4)
#define GOLLEK_HIP_ERR_NOMEM (-5)

/* ggml type ids accepted by this library (GC/core/GgmlType.java:11,16,21).  The
 * *_device mat-vec of Q5_K / Q6_K needs x 16-byte aligned and Q5_K weights
 * 4-byte aligned (else DEVICE). */
#define GOLLEK_HIP_Q4_0 2
#define GOLLEK_HIP_Q8_0 8
#define GOLLEK_HIP_Q4_K 12
#define GOLLEK_HIP_Q5_K 13 /* GC/core/GgmlType.java:22 */
#define GOLLEK_HIP_Q6_K 14 /* GC/core/GgmlType.java:23 */

/* Opaque device-resident weight matrix. */
typedef struct gollek_hip_weight gollek_hip_weight;

/* ABI version (major * 10000 + minor * 100 + patch).  No reference
 * counterpart; lets the Java binding refuse a mismatched library. */
int32_t gollek_hip_version(void);

/* Select and initialise a GPU.  Replaces the reference bridge's one-time
 * backend set-up in gollek_gguf_open (gollek_gguf_fast.cpp:692-700).
 * Calling it again with the same device is a no-op. */
int32_t gollek_hip_init(int32_t device, char *err, size_t err_len);

/* Thread-local copy of the last error message of this thread ("" if none). */
const char *gollek_hip_last_error(void);

/* Thread-local status code of this thread's last call (GOLLEK_HIP_OK after a
 * success).  Lets a caller map a NULL handle back to the exception type. */
int32_t gollek_hip_last_status(void);

/* Copy a GGUF row-major matrix (rows x cols, cols contiguous; row_bytes =
 * cols / block_size * block_bytes) from host memory to a device handle.  The
 * bytes are the tensor's bytes at dataStart + offset in the mmapped file
 * (RT/GgufTensorData.java:40, GC/loader/GGUFReader.java:30-37).  Replaces the
 * reference's prepared-matrix build at model load (RT/GgufPreparedMatrixStore
 * .java:120-127 via PRG/JavaNativeGgufBackend.java:157-180): the layout stays
 * the packed GGUF layout, only its residency changes.  NULL on failure. */
gollek_hip_weight *gollek_hip_weight_upload(int32_t type_id, const void *host_bytes,
                                            int64_t rows, int64_t cols, int64_t row_bytes,
                                            char *err, size_t err_len);

/* Wrap GGUF bytes that are already in device memory (borrowed: the caller
 * keeps ownership and must outlive the handle).  Same validation as upload. */
gollek_hip_weight *gollek_hip_weight_wrap_device(int32_t type_id, const void *device_bytes,
                                                 int64_t rows, int64_t cols,
                                                 int64_t row_bytes, char *err,
                                                 size_t err_len);

/* Build the handle's prepared mat-vec layout: a second device copy of the
 * matrix in which every workgroup's block of rows is stored superblock
 * column by column, the order the matrix-core column kernels read (Q4_K,
 * Q8_0, Q4_0 and Q5_K with K up to 16384 and at most 64 / 32 / 64 / 48 rows
 * per CU; measured 7.8 us against 8.8 us for Q4_K 14336 x 4096).  Later full mat-vecs
 * (row_count == rows) on the handle read it; every other entry point keeps
 * reading the GGUF bytes.  The layout follows the device's CU count at the
 * time of the call; a no-op (OK) for other shapes.  The copy is a snapshot:
 * a caller that rewrites a borrowed buffer (gollek_hip_weight_wrap_device)
 * after this call must call gollek_hip_weight_unprepare, or this again,
 * before the next full mat-vec.  The copy costs the matrix's bytes a second
 * time in device memory.
 * Call it before the handle's device mat-vecs start, or with none in
 * flight: a call that finds a copy for another partition frees it, and the
 * _device entry points read the copy on the caller's stream without the
 * handle's lock.
 * Replaces the reference's prepared-matrix build at model load
 * (RT/GgufPreparedMatrixStore.java:120-127 via PRG/JavaNativeGgufBackend
 * .java:157-180), which likewise keeps a prepared copy beside the raw
 * bytes.  Freed with the handle.  Device memory exhausted -> NOMEM. */
int32_t gollek_hip_weight_prepare(gollek_hip_weight *weight, char *err, size_t err_len);

/* Free the prepared copy of gollek_hip_weight_prepare, if any (OK when there
 * is none); later full mat-vecs read the GGUF bytes again, with identical
 * results.  Gives a caller the device memory back while keeping the handle,
 * as the reference's per-family prepared-cache clear keeps the raw tensor
 * (RT/GgufPreparedMatrixStore.java:129-131).  Same rule as prepare: no
 * _device call on the handle may be in flight. */
int32_t gollek_hip_weight_unprepare(gollek_hip_weight *weight, char *err, size_t err_len);

/* Keep only the prepared layout: free the handle's GGUF copy, so the packed
 * bytes are held once.  Full and prefix mat-vecs (matvec_rows, dot_row and
 * the _device form) then run the full mat-vec from the layout, so a prefix
 * or a single row returns exactly the full call's bits for its rows;
 * dequantize_rows gathers the rows' bytes back from the layout first (the
 * same bytes, so the same bits).  The GEMM entry points run up to four
 * rows of X (8-byte aligned) on the layout when K <= 4096, two up to K =
 * 16384; other GEMM shapes
 * and the MoE entry points read GGUF rows and return UNSUPPORTED for a
 * compacted handle;
 * gollek_hip_weight_unprepare rebuilds the GGUF copy (and frees the
 * layout).  Needs a prepared handle that owns its bytes: a borrowed
 * (wrap_device) buffer -> ARG, no layout -> UNSUPPORTED.  Replaces keeping
 * the raw tensor beside the prepared one (RT/GgufPreparedMatrixStore.java:
 * 120-131 keeps one prepared representation per tensor).  No _device call
 * on the handle may be in flight; the _device entries of a compacted handle
 * share temporaries of the handle (grown on demand), so they must not
 * overlap on one handle. */
int32_t gollek_hip_weight_compact(gollek_hip_weight *weight, char *err, size_t err_len);

/* Release a handle (device memory it owns, its stream and staging buffers).
 * Replaces clearPreparedMatrixCaches on backend close
 * (PRG/JavaNativeGgufBackend.java:139-143).  NULL is ignored. */
void gollek_hip_weight_free(gollek_hip_weight *weight);

/* Shape of a handle; any out pointer may be NULL. */
int32_t gollek_hip_weight_info(const gollek_hip_weight *weight, int32_t *type_id,
                               int64_t *rows, int64_t *cols, int64_t *row_bytes);

/* ---- host-buffer entry points (synchronous; the Java drop-in) ---------- */

/* Dequantize rows [row0, row0 + nrows) into dst (nrows * cols floats,
 * dst_len >= that), bit-exact with RT/GgufRowDequantizer.dequantizeRow.
 * Replaces GgufTensorOps.dequantizeRow (RT/GgufTensorOps.java:636-642) when
 * nrows == 1; row outside [0, rows) -> ARG (:652-656). */
int32_t gollek_hip_dequantize_rows(gollek_hip_weight *weight, int64_t row0, int64_t nrows,
                                   float *dst, int64_t dst_len, char *err, size_t err_len);

/* out[0] = dot(row, x).  Replaces GgufTensorOps.dotRow
 * (RT/GgufTensorOps.java:644-650): x_len >= cols (extra entries ignored),
 * row outside [0, rows) -> ARG. */
int32_t gollek_hip_dot_row(gollek_hip_weight *weight, int64_t row, const float *x,
                           int64_t x_len, float *out, char *err, size_t err_len);

/* y[r] = sum_k W[r, k] x[k] for r < row_count (a prefix of the rows).
 * Replaces GgufTensorOps.matVecRows (RT/GgufTensorOps.java:666-674) and,
 * with row_count = rows, matVec / matVecParallel (:658-664), with the
 * checks of RT/GgufMatVec.java:63-75, :196-200: row_count outside
 * [0, rows] -> ARG, y_len < row_count -> ARG, x_len < cols -> ARG,
 * row_count == 0 -> no-op. */
int32_t gollek_hip_matvec_rows(gollek_hip_weight *weight, const float *x, int64_t x_len,
                               float *y, int64_t y_len, int64_t row_count, char *err,
                               size_t err_len);

/* Y[m, n] = sum_k X[m, k] W[n, k] (Y = X W^T, the Linear convention of
 * runner/safetensor/gollek-safetensor-core/src/main/java/tech/kayys/gollek/
 * safetensor/core/tensor/AccelOps.java:370-376) for a weight of any type
 * this library takes (on bf16 matrix cores; Q6_K rows of an odd superblock
 * count on fp32 ones over their exactly dequantized values), X given as
 * m x cols bf16 bit patterns (row-major), Y m x rows fp32.  Small-M prefill
 * and batched decode.  The reference has no GGUF GEMM: it runs m independent
 * RT/GgufTensorOps.matVecRows calls (RT/GgufTensorOps.java:666-674), which
 * this replaces.  x_len < m * cols or y_len < m * rows -> ARG. */
int32_t gollek_hip_gemm_bf16(gollek_hip_weight *weight, const uint16_t *x_bf16, int64_t x_len,
                             int64_t m, float *y, int64_t y_len, char *err, size_t err_len);

/* Grouped MoE expert FFN over expert weights of any type this library takes
 * (Q4_0, Q8_0, Q4_K, Q5_K, Q6_K; gate, up and down may differ, as in Q4_K_M
 * files whose ffn_down_exps are Q6_K in some layers), stacked as GGUF stores
 * them:
 * gate and up have n_experts * inter rows of `hidden` columns, down has
 * n_experts * hidden rows of `inter` columns.  For each token t (x row-major
 * tokens x hidden) and route j < top_k (ids / weights row-major tokens x
 * top_k): out[t] += weights[t,j] * down_e(silu(gate_e x_t) * up_e x_t) with
 * e = ids[t,j], accumulated in route order; a route whose id is outside
 * [0, n_experts) or whose weight is 0 is skipped.  Replaces the per-(token,
 * route) expert loop of runner/safetensor/gollek-safetensor-engine/src/main/
 * java/tech/kayys/gollek/safetensor/engine/generation/moe/MoeForwardPass.java:
 * 217-240 with :461-472 (swigluFfn: .../engine/forward/
 * DirectForwardFfnService.java:40-61), reading each used expert once.
 * Other weight types -> UNSUPPORTED; gate rows not a multiple of n_experts,
 * shapes that disagree, or tokens * top_k above 2^24 -> ARG. */
int32_t gollek_hip_moe_grouped(gollek_hip_weight *gate, gollek_hip_weight *up,
                               gollek_hip_weight *down, int64_t n_experts, const float *x,
                               int64_t tokens, const int32_t *ids, const float *weights,
                               int64_t top_k, float *out, int64_t out_len, char *err,
                               size_t err_len);

/* Device workspace bytes gollek_hip_moe_grouped_device needs. */
int64_t gollek_hip_moe_workspace_bytes(int64_t tokens, int64_t top_k, int64_t hidden,
                                       int64_t inter, int64_t n_experts);

/* ---- device-buffer entry points (asynchronous on `stream`) ------------- */
/* `stream` is a hipStream_t passed as void* (NULL = the null stream).  All
 * pointers are device pointers.  Same semantics as the host versions. */

int32_t gollek_hip_dequantize_rows_device(gollek_hip_weight *weight, int64_t row0,
                                          int64_t nrows, float *dst, void *stream, char *err,
                                          size_t err_len);

int32_t gollek_hip_matvec_device(gollek_hip_weight *weight, const float *x, float *y,
                                 int64_t row_count, void *stream, char *err, size_t err_len);

/* Shapes whose output tiles leave CUs idle (few 128 x 128 tiles for the
 * chip) are split over K into partial tiles held in a workspace of the
 * handle, allocated at the first such call (below 16 MiB on 256 CUs) and
 * freed with the handle; splitting calls on one handle share it and must not
 * overlap (calls on different handles may).  A y that is not 16-byte aligned
 * runs unsplit. */
int32_t gollek_hip_gemm_bf16_device(gollek_hip_weight *weight, const uint16_t *x_bf16, int64_t m,
                                    float *y, void *stream, char *err, size_t err_len);

/* gollek_hip_gemm_bf16_device without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code
 * under HIP graph capture, tight serving loops).  The split-K partial tiles
 * go to a static per-GPU scratch of 16 MiB (held from library load until the
 * process ends; enough for every shape on a 256-CU MI355X) instead of the
 * handle's lazily allocated workspace; a shape whose splits would need more
 * is split less, down to none.  All calls on one GPU share that scratch, so
 * calls that overlap on a GPU race.  Same checks and results as
 * gollek_hip_gemm_bf16_device. */
int32_t gollek_hip_gemm_bf16_device_noalloc(gollek_hip_weight *weight, const uint16_t *x_bf16,
                                            int64_t m, float *y, void *stream, char *err,
                                            size_t err_len);

/* `workspace` (device, workspace_bytes >= gollek_hip_moe_workspace_bytes) is
 * scratch owned by the caller; calls sharing one workspace must not overlap. */
int32_t gollek_hip_moe_grouped_device(gollek_hip_weight *gate, gollek_hip_weight *up,
                                      gollek_hip_weight *down, int64_t n_experts, const float *x,
                                      const int32_t *ids, const float *weights, int64_t tokens,
                                      int64_t top_k, float *out, void *workspace,
                                      int64_t workspace_bytes, void *stream, char *err,
                                      size_t err_len);

/* ---- MoE router and the routed block ------------------------------------ */
/* SFE/ = runner/safetensor/gollek-safetensor-engine/src/main/java/tech/kayys/
 * gollek/safetensor/engine/. */

/* Router scoring (SFE/generation/moe/MoeForwardPass.java:174-197): the
 * reference picks sigmoid when the model type contains "qwen" or "moe",
 * softmax otherwise; the caller passes that choice. */
#define GOLLEK_HIP_ROUTER_SOFTMAX 0
#define GOLLEK_HIP_ROUTER_SIGMOID 1

/* Per token t (logits row-major tokens x n_experts, the router linear's
 * output): probabilities by `scoring` (sigmoid 1 / (1 + exp(-l)); softmax
 * exp(l - max) / sum with exp in double and float sums in expert order),
 * then the top_k experts in descending probability order, ties in index
 * order, and their probabilities divided by their float sum when that sum
 * is > 0 -> ids / weights (row-major tokens x top_k).  Ranks past n_experts
 * get id 0, weight 0.  Replaces MoeForwardPass.java:174-203 with selectTopK
 * (:286-306), bit for bit.  n_experts or top_k outside [1, 4096], an unknown
 * scoring -> ARG.  Synchronous; allocates device memory per call (the
 * _device variant does not). */
int32_t gollek_hip_moe_select_topk(const float *logits, int64_t tokens, int64_t n_experts,
                                   int64_t top_k, int32_t scoring, int32_t *ids, float *weights,
                                   char *err, size_t err_len);
int32_t gollek_hip_moe_select_topk_device(const float *logits, int64_t tokens, int64_t n_experts,
                                          int64_t top_k, int32_t scoring, int32_t *ids,
                                          float *weights, void *stream, char *err,
                                          size_t err_len);

/* The routed MoE block: gollek_hip_moe_select_topk on `logits` followed by
 * gollek_hip_moe_grouped with the ids and weights it chose, on one stream
 * (MoeForwardPass.java:174-240 after the router linear).  The shared expert
 * (:240-247) follows with gollek_hip_moe_shared_expert on the same `out`.
 * Checks of both calls apply. */
int32_t gollek_hip_moe_block(gollek_hip_weight *gate, gollek_hip_weight *up,
                             gollek_hip_weight *down, int64_t n_experts, const float *x,
                             int64_t tokens, const float *logits, int64_t top_k, int32_t scoring,
                             float *out, int64_t out_len, char *err, size_t err_len);
/* Device variant: also writes the chosen ids / weights (device, tokens x
 * top_k) and takes the grouped FFN's workspace from the caller
 * (gollek_hip_moe_workspace_bytes; calls sharing it must not overlap). */
int32_t gollek_hip_moe_block_device(gollek_hip_weight *gate, gollek_hip_weight *up,
                                    gollek_hip_weight *down, int64_t n_experts, const float *x,
                                    const float *logits, int64_t tokens, int64_t top_k,
                                    int32_t scoring, int32_t *ids, float *weights, float *out,
                                    void *workspace, int64_t workspace_bytes, void *stream,
                                    char *err, size_t err_len);

/* The shared expert, added to the routed output of the same tokens
 * (SFE/generation/moe/MoeForwardPass.java:240-247 with runSharedExpert
 * :418-426 and resolveSharedExpertGate :428-442): for each token t
 *   out[t] = out[t] + g_t * y_t   (the product rounded, then the sum),
 *   y_t = down(silu(gate x_t) * (up x_t)),
 *   g_t = 1 / (1 + (float)exp(-s_t)) with exp in double, s_t = x_t . gate_inp
 *         rounded to float (gate_inp: `hidden` floats, the shared_expert_gate
 *         row); g_t = 1 when gate_inp is NULL (the reference's missing gate).
 * gate / up: inter x hidden, down: hidden x inter, of any types
 * gollek_hip_moe_grouped takes.  Errors as gollek_hip_moe_grouped with one
 * expert (x and out NULL -> NULL; out_len < tokens * hidden -> ARG). */
int32_t gollek_hip_moe_shared_expert(gollek_hip_weight *gate, gollek_hip_weight *up,
                                     gollek_hip_weight *down, const float *gate_inp, const float *x,
                                     int64_t tokens, float *out, int64_t out_len, char *err,
                                     size_t err_len);
/* Device workspace bytes gollek_hip_moe_shared_expert_device needs. */
int64_t gollek_hip_moe_shared_workspace_bytes(int64_t tokens, int64_t hidden, int64_t inter);
/* Device variant (x, gate_inp, out on the device; `workspace` as for
 * gollek_hip_moe_grouped_device, >= gollek_hip_moe_shared_workspace_bytes). */
int32_t gollek_hip_moe_shared_expert_device(gollek_hip_weight *gate, gollek_hip_weight *up,
                                            gollek_hip_weight *down, const float *gate_inp, const float *x,
                                            int64_t tokens, float *out, void *workspace,
                                            int64_t workspace_bytes, void *stream, char *err,
                                            size_t err_len);

/* ---- GGUF files --------------------------------------------------------- */
/* GC/ = runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf/. */

/* Opaque parsed GGUF file (a read-only mapping of it plus its tensor table). */
typedef struct gollek_hip_gguf gollek_hip_gguf;

/* Maps `path` read-only and parses the header, the metadata (skipped, except
 * general.alignment, default 32) and the tensor infos; needs no GPU.
 * Replaces GC/loader/GGUFReader.java:28-37 (open + mmap) with
 * GC/loader/GGUFParser.java:17-105 (parse).  Returns NULL with the status
 * (gollek_hip_last_status) and message set: bad magic -> ARG "Not a valid
 * GGUF file"; a metadata type outside 0..12 -> UNSUPPORTED "Unsupported GGUF
 * KV type: N at pos P"; a tensor type without a GGUF block layout or an
 * element count that is not a multiple of its block -> UNSUPPORTED
 * "Unsupported or misaligned GGUF tensor type T with N element(s)"; a
 * truncated file, a negative or oversized length or count, more than 8
 * dimensions, a non-numeric or non-positive general.alignment -> ARG. */
gollek_hip_gguf *gollek_hip_gguf_open(const char *path, char *err, size_t err_len);

/* Unmaps the file and frees its upload buffers.  Weight handles uploaded from
 * it stay valid.  NULL is a no-op. */
void gollek_hip_gguf_close(gollek_hip_gguf *file);

/* Header facts: format version, tensor and metadata counts, the alignment
 * used, the absolute offset of the tensor data (GGUFModel.dataStart,
 * GC/loader/GGUFParser.java:57-62) and the file size.  Any pointer may be NULL. */
int32_t gollek_hip_gguf_info(const gollek_hip_gguf *file, int32_t *version, int64_t *n_tensors,
                             int64_t *n_kv, int64_t *alignment, int64_t *data_start,
                             int64_t *file_bytes);

/* Tensor `index` in file order (GC/loader/GGUFTensorInfo.java:8-14): name
 * (NUL-terminated, truncated to name_len - 1), ggml type id, dimension count,
 * dims[0..7] (dims[0] = the contiguous one; unused entries 1), offset from
 * the data start and size in bytes.  Index out of range -> ARG.  Output
 * pointers may be NULL. */
int32_t gollek_hip_gguf_tensor(const gollek_hip_gguf *file, int64_t index, char *name,
                               size_t name_len, int32_t *type_id, int32_t *n_dims, int64_t *dims,
                               int64_t *offset, int64_t *size_bytes);

/* Index of the first tensor named `name` (GGUFModel.tensors lookup by name),
 * or -1. */
int64_t gollek_hip_gguf_find(const gollek_hip_gguf *file, const char *name);

/* Copies tensor `index` to a new device weight handle on the current device
 * (rows = product of dims[1..], cols = dims[0]), through pinned staging
 * buffers the file object keeps.  Replaces the byte slice of
 * GC/runtime/GgufTensorData.java:97-104 followed by gollek_hip_weight_upload:
 * bytes outside the file -> ARG "Tensor data range is outside model segment:
 * NAME"; then the validation of gollek_hip_weight_upload (types other than
 * Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K -> UNSUPPORTED).  Free the handle with
 * gollek_hip_weight_free.  Thread-safe; uploads from one file object
 * serialise on its staging buffers. */
gollek_hip_weight *gollek_hip_gguf_upload(gollek_hip_gguf *file, int64_t index, char *err,
                                          size_t err_len);

#ifdef __cplusplus
}
#endif
#endif /* GOLLEK_HIP_H */
