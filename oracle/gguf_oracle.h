/*
 * gguf_oracle.h -- CPU oracle for the GGUF quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY.  This is a plain-C restatement of gollek's Java
 * raw route (runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/
 * gguf/runtime/, abbreviated RT/ below).  It is the checker the HIP library is
 * compared against and the CPU baseline that bench.py reports beside the GPU.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may
 * load it.  The product library (gollek_amd/) never links, loads or calls it.
 *
 * Parity pinning (what fixes each function independently of this file):
 *   go_f16_to_f32        exhaustive check against numpy's IEEE half decoder
 *                        (all 65536 codes) + the reference fp16 special-value
 *                        fixture (TST/GgufF16SpecialTest.java:18-44).
 *   go_k4_scale_min      round trip against the generator's inverse packer
 *                        over random codes + the reference Q4_K fixtures.
 *   go_dequantize_row    reference closed-form fixtures (TST/GgufQ4KTest,
 *                        GgufQ4KRawTest lane-order rows, GgufQ4KMixTest,
 *                        GgufQ32Test, GgufQ32Q4LaneTest, GgufQ8Test) and a
 *                        numpy restatement of the textbook block formulas.
 *   go_dot_row /         reference closed-form dots (384, 128, 16/48, 32/64,
 *   go_matvec_rows       +-2464, -264, lane-order dots) and an fp64 dot over
 *                        the bit-exact dequantized rows at 1e-3.
 *   go_dequantize_row    Q5_K / Q6_K: the reference's lane-order fixtures
 *   (Q5_K, Q6_K)         (TST/GgufQ5LaneFx, GgufQ5CalcFx, GgufQ6LaneFx,
 *                        GgufQ5KOffTest) and the numpy restatement of the
 *                        ggml block formulas (tests/npref.py).
 *   go_dot_row /         Q5_K / Q6_K: the same lane-order fixtures' dots at
 *   go_matvec_rows       0.0; closed forms of constant blocks (every code and
 *   (Q5_K, Q6_K)         x equal: the row sum is a product of exact
 *                        integers, met by every walker); the no-min,
 *                        inline, direct and group-sum walkers against each
 *                        other and against an fp64 dot at 1e-4; and planted
 *                        mistakes (a high bit from the wrong plane, a lost
 *                        -32, a scale from the wrong half) that those checks
 *                        catch (tests/test_oracle.py).
 *   go_moe_select_topk   closed forms (uniform logits: ids 0..k-1 by the
 *                        stable tie order, weights 1/k; distinct logits:
 *                        numpy's stable descending argsort and fp64
 *                        probabilities; a NaN probability ranks first and
 *                        skips the renormalisation; k past the expert count
 *                        pads id 0 / weight 0; all-zero sigmoid weights stay
 *                        0) in tests/test_oracle.py.
 * The fp32 rounding order of the Java Vector-API kernels (FloatVector lane
 * reductions) cannot be reproduced without a JVM; the scalar Java loops are
 * restated instead, so GEMV parity is tolerance-based (1e-3), as specified.
 */
#ifndef GOLLEK_GGUF_ORACLE_H
#define GOLLEK_GGUF_ORACLE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (GC/core/GgmlType.java:11,16,21). */
enum { GO_Q4_0 = 2, GO_Q8_0 = 8, GO_Q4_K = 12, GO_Q5_K = 13, GO_Q6_K = 14 };

/* Status codes shared with the oracle's Python wrapper. */
enum {
    GO_OK = 0,
    GO_ERR_ARG = -2,        /* IllegalArgumentException in the reference */
    GO_ERR_UNSUPPORTED = -3 /* UnsupportedOperationException */
};

int go_block_size(int type_id);  /* elements per block, 0 if unsupported */
int go_block_bytes(int type_id); /* bytes per block, 0 if unsupported */
/* Row bytes for `cols` columns; -1 if unsupported or cols % block != 0. */
int64_t go_row_bytes(int type_id, int64_t cols);

float go_f16_to_f32(uint16_t bits);
void go_f16_to_f32_n(const uint16_t *bits, int64_t n, float *out);
void go_k4_scale_min(const uint8_t *scales12, int j, int *sc, int *m);

/* Bit-exact dequantization of one row of `cols` elements. */
int go_dequantize_row(int type_id, const uint8_t *row, int64_t cols, float *dst);
/* Dequantize rows [row0, row0+nrows) of a row-major matrix. */
int go_dequantize_rows(int type_id, const uint8_t *data, int64_t row_bytes,
                       int64_t cols, int64_t row0, int64_t nrows, float *dst);

/* Single-row dot product in the Java raw single-row order. */
int go_dot_row(int type_id, const uint8_t *row, int64_t cols, const float *x,
               float *out);

/* Mat-vec over the first row_count rows, in the Java raw multi-row order.
 * threads <= 0 means "all host cores"; threads == 1 is serial.  The chunking
 * follows RT/GgufParallelConfig.java:24-72 (2 chunks per thread, parallel
 * only when row_count * cols >= 131072). */
int go_matvec_rows(int type_id, const uint8_t *data, int64_t rows, int64_t cols,
                   int64_t row_bytes, const float *x, float *y,
                   int64_t row_count, int threads);

/* Number of host threads go_matvec_rows uses when threads <= 0. */
int go_default_threads(void);

/* Per-32 and per-16 group sums of x (RT/GgufSum.java:30-66), sequential
 * order. */
void go_group_sums32(const float *x, int64_t cols, float *sums);
void go_group_sums16(const float *x, int64_t cols, float *sums);

/* Whether any of the first row_count rows of a Q4_K matrix has an active min
 * (RT/GgufKMeta.java:115-181). */
int go_q4k_rows_have_mins(const uint8_t *data, int64_t row_bytes, int64_t cols,
                          int64_t row_count);
/* The same for Q4_K or Q5_K (type_id 12 or 13); GO_ERR_UNSUPPORTED else. */
int go_k_rows_have_mins(int type_id, const uint8_t *data, int64_t row_bytes, int64_t cols,
                        int64_t row_count);

/* MoE router (runner/safetensor/gollek-safetensor-engine/src/main/java/tech/
 * kayys/gollek/safetensor/engine/generation/moe/MoeForwardPass.java:174-203,
 * 286-306): logits [tokens, n_experts] -> sigmoid (sigmoid != 0) or softmax
 * probabilities, top_k by a stable descending Float.compare sort, weights
 * renormalised by their float sum when it is > 0 -> ids / weights
 * [tokens, top_k] (ranks past n_experts: id 0, weight 0). */
int go_moe_select_topk(const float *logits, int64_t tokens, int64_t n_experts, int64_t top_k,
                       int sigmoid, int32_t *ids, float *weights);

#ifdef __cplusplus
}
#endif
#endif
