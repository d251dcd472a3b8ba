/*
 * gguf_oracle.c -- CPU oracle for the GGUF quantized linear-layer path.
 *
 * TEST INFRASTRUCTURE ONLY (see gguf_oracle.h for who may load it and how
 * each function is pinned).  Restates gollek's Java raw route; every function
 * cites the Java it follows.  RT/ abbreviates
 *   runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf/runtime/
 *
 * Must be compiled without floating-point contraction (-ffp-contract=off) and
 * without -ffast-math: Java evaluates every float operation with one IEEE
 * rounding and no fused multiply-add, and the dequantizers are bit-exact.
 */
#include "gguf_oracle.h"

#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

#define QK_K 256

/* GO_PLANT n (n > 0) builds a copy with one planted mistake, for the tests
 * that show the oracle's checks catch it (never set in the built oracle):
 *   1  Q5_K low codes take their high bit from the high codes' plane
 *   2  Q6_K direct dots drop the -32 offset
 *   3  Q6_K second-half groups use the first half's scales
 *   4  Q6_K group-sum dots subtract the wrong 16-element x sum
 *   5  Q4_K / Q5_K second sub-block of a chunk uses the first one's min */
#ifndef GO_PLANT
#define GO_PLANT 0
#endif

/* ---- format geometry (GC/core/GgmlType.java:11,16,21,70-81) ------------ */

int go_block_size(int type_id) {
    switch (type_id) {
    case GO_Q4_0: return 32;
    case GO_Q8_0: return 32;
    case GO_Q4_K: return QK_K;
    case GO_Q5_K: return QK_K;
    case GO_Q6_K: return QK_K;
    default: return 0;
    }
}

int go_block_bytes(int type_id) {
    switch (type_id) {
    case GO_Q4_0: return 18;
    case GO_Q8_0: return 34;
    case GO_Q4_K: return 144;
    case GO_Q5_K: return 176;
    case GO_Q6_K: return 210;
    default: return 0;
    }
}

int64_t go_row_bytes(int type_id, int64_t cols) {
    int bs = go_block_size(type_id);
    if (bs == 0 || cols < 0 || cols % bs != 0) return -1;
    return (cols / bs) * (int64_t)go_block_bytes(type_id);
}

static uint16_t rd16(const uint8_t *p) { return (uint16_t)(p[0] | (p[1] << 8)); }

/* ---- fp16 decode (RT/GgufQuantTables.java:142-164) ---------------------- */

float go_f16_to_f32(uint16_t bits) {
    uint32_t sign = (bits >> 15) & 1u;
    uint32_t exponent = (bits >> 10) & 0x1Fu;
    uint32_t mantissa = bits & 0x3FFu;
    if (exponent == 0) {
        if (mantissa == 0) return sign ? -0.0f : 0.0f;
        /* scalb(mantissa / 1024, -14) == mantissa * 2^-24, exact in fp32 */
        float value = ldexpf((float)mantissa, -24);
        return sign ? -value : value;
    }
    if (exponent == 31) {
        if (mantissa == 0) return sign ? -INFINITY : INFINITY;
        /* The reference returns Float.NaN: the canonical quiet NaN. */
        uint32_t nan_bits = 0x7FC00000u;
        float nan_value;
        memcpy(&nan_value, &nan_bits, 4);
        return nan_value;
    }
    uint32_t f = (sign << 31) | ((exponent + 112u) << 23) | (mantissa << 13);
    float out;
    memcpy(&out, &f, 4);
    return out;
}

void go_f16_to_f32_n(const uint16_t *bits, int64_t n, float *out) {
    for (int64_t i = 0; i < n; i++) out[i] = go_f16_to_f32(bits[i]);
}

/* ---- K-quant 6-bit scale/min unpack (RT/GgufKQuantLayout.java:37-65) ---- */

void go_k4_scale_min(const uint8_t *b, int j, int *sc, int *m) {
    if (j < 4) {
        *sc = b[j] & 63;
        *m = b[j + 4] & 63;
    } else {
        *sc = (b[j + 4] & 0x0F) | ((b[j - 4] >> 6) << 4);
        *m = (b[j + 4] >> 4) | ((b[j] >> 6) << 4);
    }
}

/* RT/GgufKQuantLayout.java:67-69 */
static float min_contribution(float dmin, int code) {
    return code == 0 ? 0.0f : dmin * (float)code;
}

/* ---- dequantizers (bit-exact) ------------------------------------------ */

/* RT/GgufRowDequantizer.java:141-152 -> RT/GgufBlockDequantizer.java:230-264 */
static void dequant_q8_0_block(const uint8_t *blk, float *y) {
    float d = go_f16_to_f32(rd16(blk));
    const int8_t *q = (const int8_t *)(blk + 2);
    for (int i = 0; i < 32; i++) y[i] = (float)q[i] * d;
}

/* RT/GgufBlockDequantizer.java:32-36 and :365-414 (zero point 8, bias +0.0f) */
static void dequant_q4_0_block(const uint8_t *blk, float *y) {
    float d = go_f16_to_f32(rd16(blk));
    const uint8_t *q = blk + 2;
    for (int i = 0; i < 16; i++) {
        y[i] = (float)((q[i] & 0x0F) - 8) * d + 0.0f;
        y[16 + i] = (float)((q[i] >> 4) - 8) * d + 0.0f;
    }
}

/* RT/GgufKBlockDequantizer.java:31-88 */
static void dequant_q4_k_block(const uint8_t *blk, float *y) {
    float d = go_f16_to_f32(rd16(blk));
    float dmin = go_f16_to_f32(rd16(blk + 2));
    const uint8_t *scales = blk + 4;
    const uint8_t *qs = blk + 16;
    for (int c = 0; c < 4; c++) {
        int sc1, mc1, sc2, mc2;
        go_k4_scale_min(scales, 2 * c, &sc1, &mc1);
        go_k4_scale_min(scales, 2 * c + 1, &sc2, &mc2);
        float d1 = d * (float)sc1;
        float d2 = d * (float)sc2;
        float m1 = 0.0f, m2 = 0.0f;
        if (!(dmin == 0.0f)) {
            m1 = min_contribution(dmin, mc1);
            m2 = min_contribution(dmin, mc2);
        }
        const uint8_t *q = qs + 32 * c;
        for (int i = 0; i < 32; i++) {
            y[64 * c + i] = d1 * (float)(q[i] & 0x0F) - m1;
            y[64 * c + 32 + i] = d2 * (float)(q[i] >> 4) - m2;
        }
    }
}

/* RT/GgufRowDequantizer.java:29-276 (Q4_0 :97-107, Q8_0 :141-152,
 * Q4_K :242-252, unsupported :275) */
/* RT/GgufKBlockDequantizer.java:91-170: Q5_K.  Chunk c (64 elements) uses
 * sub-blocks 2c, 2c+1, quants 48 + 32c.., and high-bit masks 1 << 2c,
 * 2 << 2c over qh[0..32); values fl(fl(d1 * q) - m1), the min rules of Q4_K. */
static void dequant_q5_k_block(const uint8_t *blk, float *y) {
    const float d = go_f16_to_f32(rd16(blk));
    const float dmin = go_f16_to_f32(rd16(blk + 2));
    const uint8_t *qh = blk + 16;
    for (int c = 0; c < 4; c++) {
        int sc1, m1c, sc2, m2c;
        go_k4_scale_min(blk + 4, 2 * c, &sc1, &m1c);
        go_k4_scale_min(blk + 4, 2 * c + 1, &sc2, &m2c);
        const float d1 = d * (float)sc1, d2 = d * (float)sc2;
        float m1 = 0.0f, m2 = 0.0f;
        if (dmin != 0.0f) {
            m1 = min_contribution(dmin, m1c);
            m2 = min_contribution(dmin, m2c);
        }
        const uint8_t *qs = blk + 48 + 32 * c;
        const int mlo = 1 << (2 * c), mhi = 2 << (2 * c);
        for (int i = 0; i < 32; i++) {
            const int lo = (qs[i] & 0x0F) + ((qh[i] & mlo) != 0 ? 16 : 0);
            const int hi = (qs[i] >> 4) + ((qh[i] & mhi) != 0 ? 16 : 0);
            y[64 * c + i] = d1 * (float)lo - m1;
            y[64 * c + 32 + i] = d2 * (float)hi - m2;
        }
    }
}

/* RT/GgufKBlockDequantizer.java:319-432: Q6_K, d at byte 208; per 128-element
 * half: ql 64 bytes, qh 32 bytes, 8 int8 scales; values fl(fl(d * sc) * (q - 32)). */
static void dequant_q6_k_block(const uint8_t *blk, float *y) {
    const float d = go_f16_to_f32(rd16(blk + 208));
    for (int h = 0; h < 2; h++) {
        const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
        const int8_t *sc = (const int8_t *)(blk + 192 + 8 * h);
        float *o = y + 128 * h;
        for (int half = 0; half < 2; half++) {
            const float s1 = d * (float)sc[half], s2 = d * (float)sc[half + 2];
            const float s3 = d * (float)sc[half + 4], s4 = d * (float)sc[half + 6];
            for (int i = 16 * half; i < 16 * half + 16; i++) {
                const int a = ql[i], b = ql[32 + i], hb = qh[i];
                o[i] = s1 * (float)(((a & 0x0F) | ((hb & 0x03) << 4)) - 32);
                o[32 + i] = s2 * (float)(((b & 0x0F) | (((hb >> 2) & 0x03) << 4)) - 32);
                o[64 + i] = s3 * (float)(((a >> 4) | (((hb >> 4) & 0x03) << 4)) - 32);
                o[96 + i] = s4 * (float)(((b >> 4) | (((hb >> 6) & 0x03) << 4)) - 32);
            }
        }
    }
}

int go_dequantize_row(int type_id, const uint8_t *row, int64_t cols, float *dst) {
    int bs = go_block_size(type_id);
    if (bs == 0) return GO_ERR_UNSUPPORTED;
    if (cols % bs != 0) return GO_ERR_ARG;
    int bb = go_block_bytes(type_id);
    int64_t blocks = cols / bs;
    for (int64_t b = 0; b < blocks; b++) {
        const uint8_t *blk = row + b * bb;
        float *y = dst + b * bs;
        if (type_id == GO_Q8_0) dequant_q8_0_block(blk, y);
        else if (type_id == GO_Q4_0) dequant_q4_0_block(blk, y);
        else if (type_id == GO_Q5_K) dequant_q5_k_block(blk, y);
        else if (type_id == GO_Q6_K) dequant_q6_k_block(blk, y);
        else dequant_q4_k_block(blk, y);
    }
    return GO_OK;
}

int go_dequantize_rows(int type_id, const uint8_t *data, int64_t row_bytes,
                       int64_t cols, int64_t row0, int64_t nrows, float *dst) {
    for (int64_t r = 0; r < nrows; r++) {
        int rc = go_dequantize_row(type_id, data + (row0 + r) * row_bytes, cols,
                                   dst + r * cols);
        if (rc != GO_OK) return rc;
    }
    return GO_OK;
}

/* ---- Q8_0 raw dot (RT/GgufQ8RawDot.java:137-184, :783-825) -------------- */

static float q8_unscaled_block(const uint8_t *qb, const float *x) {
    const int8_t *q = (const int8_t *)qb;
    float lane[4];
    for (int k = 0; k < 4; k++) {
        float s = (float)q[k] * x[k] + (float)q[k + 4] * x[k + 4];
        for (int p = 1; p < 4; p++) {
            int o = 8 * p + k;
            s += (float)q[o] * x[o] + (float)q[o + 4] * x[o + 4];
        }
        lane[k] = s;
    }
    return lane[0] + lane[1] + lane[2] + lane[3];
}

static float dot_q8_0(const uint8_t *row, int64_t cols, const float *x) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    int64_t blocks = cols / 32, b = 0;
    for (; b + 4 <= blocks; b += 4) {
        const uint8_t *p = row + b * 34;
        const float *v = x + b * 32;
        s0 += go_f16_to_f32(rd16(p)) * q8_unscaled_block(p + 2, v);
        s1 += go_f16_to_f32(rd16(p + 34)) * q8_unscaled_block(p + 36, v + 32);
        s2 += go_f16_to_f32(rd16(p + 68)) * q8_unscaled_block(p + 70, v + 64);
        s3 += go_f16_to_f32(rd16(p + 102)) * q8_unscaled_block(p + 104, v + 96);
    }
    float sum = s0 + s1 + s2 + s3;
    for (; b < blocks; b++) {
        const uint8_t *p = row + b * 34;
        float d = go_f16_to_f32(rd16(p));
        sum += d * q8_unscaled_block(p + 2, x + b * 32);
    }
    return sum;
}

/* ---- Q4_0 raw dot (RT/GgufQ32RawDot.java:33-66, :341-348, :427-462) ------ */

static float q4_0_nibble_pair(const uint8_t *q, const float *x, int i) {
    return (float)((q[i] & 0x0F) - 8) * x[i] + (float)((q[i] >> 4) - 8) * x[16 + i];
}

static float q4_0_unscaled_block(const uint8_t *q, const float *x) {
    float lane[4];
    for (int k = 0; k < 4; k++) {
        lane[k] = q4_0_nibble_pair(q, x, k) + q4_0_nibble_pair(q, x, k + 4)
                + q4_0_nibble_pair(q, x, k + 8) + q4_0_nibble_pair(q, x, k + 12);
    }
    return lane[0] + lane[1] + lane[2] + lane[3];
}

static float q4_0_block(const uint8_t *p, const float *x) {
    float d = go_f16_to_f32(rd16(p));
    return d * q4_0_unscaled_block(p + 2, x);
}

static float dot_q4_0(const uint8_t *row, int64_t cols, const float *x) {
    float s0 = 0.0f, s1 = 0.0f, s2 = 0.0f, s3 = 0.0f;
    int64_t blocks = cols / 32, b = 0;
    for (; b + 4 <= blocks; b += 4) {
        const uint8_t *p = row + b * 18;
        const float *v = x + b * 32;
        s0 += q4_0_block(p, v);
        s1 += q4_0_block(p + 18, v + 32);
        s2 += q4_0_block(p + 36, v + 64);
        s3 += q4_0_block(p + 54, v + 96);
    }
    float sum = s0 + s1 + s2 + s3;
    for (; b < blocks; b++) sum += q4_0_block(row + b * 18, x + b * 32);
    return sum;
}

/* ---- Q4_K / Q5_K raw dots (RT/GgufQ4RawDot.java, RT/GgufQ5RawDot.java) ---
 * Q5_K is Q4_K's block with 32 bytes of high bits placed before the quants
 * (176 bytes: d, dmin, 12 scale bytes, qh[32], qs[128]).  Its code for
 * element i of chunk c is the Q4_K nibble plus 16 x bit 2c (low nibbles) or
 * bit 2c+1 (high nibbles) of qh[i]; every loop, accumulator and branch of the
 * Java Q5_K dots is otherwise that of the Q4_K ones (RT/GgufQ5RawDot.java:
 * 37-172 beside RT/GgufQ4RawDot.java:37-146, :174-329 beside :148-329,
 * :393-795 beside :331-674), so one set of functions serves both. */

typedef struct {
    int bytes; /* block bytes */
    int qs;    /* offset of the 128 quant bytes */
    int qh;    /* offset of the 32 high-bit bytes, -1 without */
} kfmt;

static const kfmt KF_Q4 = {144, 16, -1};
static const kfmt KF_Q5 = {176, 48, 16};

/* Partial dots of one 64-element chunk c: the low codes of the 32 bytes pair
 * with x[0..32), the high codes with x[32..64).  Accumulated in groups of 8
 * exactly as the Java loops do (RT/GgufQ4RawDot.java:83-131, :642-668;
 * RT/GgufQ5RawDot.java:87-153, :740-790: eight products summed left to
 * right, then added to the chunk's accumulator). */
static void k_chunk_dots(const uint8_t *blk, const kfmt *f, int c, const float *x,
                         float *qd1, float *qd2, float *vs1, float *vs2) {
    const uint8_t *q = blk + f->qs + 32 * c;
    const uint8_t *qh = f->qh >= 0 ? blk + f->qh : NULL;
    float a1 = 0.0f, a2 = 0.0f, v1 = 0.0f, v2 = 0.0f;
    for (int i = 0; i < 32; i += 8) {
        float t1 = 0.0f, t2 = 0.0f, u1 = 0.0f, u2 = 0.0f;
        for (int k = 0; k < 8; k++) {
            int lo = q[i + k] & 0x0F, hi = q[i + k] >> 4;
            if (qh) {
                lo += ((qh[i + k] >> (GO_PLANT == 1 ? 2 * c + 1 : 2 * c)) & 1) << 4;
                hi += ((qh[i + k] >> (2 * c + 1)) & 1) << 4;
            }
            float p1 = (float)lo * x[i + k], p2 = (float)hi * x[32 + i + k];
            t1 = k ? t1 + p1 : p1;
            t2 = k ? t2 + p2 : p2;
            u1 = k ? u1 + x[i + k] : x[i + k];
            u2 = k ? u2 + x[32 + i + k] : x[32 + i + k];
        }
        a1 += t1;
        a2 += t2;
        v1 += u1;
        v2 += u2;
    }
    *qd1 = a1;
    *qd2 = a2;
    if (vs1) *vs1 = v1;
    if (vs2) *vs2 = v2;
}

/* dotRowQ4K / dotRowQ5K: single row, inline vector sums
 * (RT/GgufQ4RawDot.java:37-146, RT/GgufQ5RawDot.java:37-172). */
static float dot_k_inline(const kfmt *f, const uint8_t *row, int64_t cols, const float *x) {
    float sum = 0.0f;
    int64_t blocks = cols / QK_K;
    for (int64_t b = 0; b < blocks; b++) {
        const uint8_t *blk = row + b * f->bytes;
        const float *v = x + b * QK_K;
        float d = go_f16_to_f32(rd16(blk));
        float dmin = go_f16_to_f32(rd16(blk + 2));
        int has_block_mins = !(dmin == 0.0f);
        for (int c = 0; c < 4; c++) {
            int sc1, mc1, sc2, mc2;
            go_k4_scale_min(blk + 4, 2 * c, &sc1, &mc1);
            go_k4_scale_min(blk + 4, 2 * c + 1, &sc2, &mc2);
            float d1 = d * (float)sc1;
            float d2 = d * (float)sc2;
            int min1 = has_block_mins ? mc1 : 0;
            int min2 = has_block_mins ? (GO_PLANT == 5 ? mc1 : mc2) : 0;
            float qd1, qd2, vs1, vs2;
            k_chunk_dots(blk, f, c, v + 64 * c, &qd1, &qd2, &vs1, &vs2);
            sum += d1 * qd1 + d2 * qd2;
            if (min1 != 0) sum -= dmin * (float)min1 * vs1;
            if (min2 != 0) sum -= dmin * (float)min2 * vs2;
        }
    }
    return sum;
}

/* dotRowQ4KNoMinBlock (RT/GgufQ4RawDot.java:255-329) /
 * dotRowQ5KNoMinBlock (RT/GgufQ5RawDot.java:276-391) */
static float k_nomin_block(const kfmt *f, const uint8_t *blk, const float *v) {
    float d = go_f16_to_f32(rd16(blk));
    float part[4];
    for (int c = 0; c < 4; c++) {
        int sc1, mc1, sc2, mc2;
        go_k4_scale_min(blk + 4, 2 * c, &sc1, &mc1);
        go_k4_scale_min(blk + 4, 2 * c + 1, &sc2, &mc2);
        float d1 = d * (float)sc1;
        float d2 = d * (float)sc2;
        float qd1, qd2;
        k_chunk_dots(blk, f, c, v + 64 * c, &qd1, &qd2, NULL, NULL);
        part[c] = d1 * qd1 + d2 * qd2;
    }
    return part[0] + part[1] + part[2] + part[3];
}

/* dotRowQ4KGroupSumBlock / ...SuperBlock (RT/GgufQ4RawDot.java:531-674),
 * dotRowQ5KGroupSumBlock / ...SuperBlock (RT/GgufQ5RawDot.java:604-795) */
static float k_groupsum_block(const kfmt *f, const uint8_t *blk, const float *v,
                              const float *gs) {
    float d = go_f16_to_f32(rd16(blk));
    float dmin = go_f16_to_f32(rd16(blk + 2));
    int has_block_mins = !(dmin == 0.0f);
    float part[4];
    for (int c = 0; c < 4; c++) {
        int sc1, mc1, sc2, mc2;
        go_k4_scale_min(blk + 4, 2 * c, &sc1, &mc1);
        go_k4_scale_min(blk + 4, 2 * c + 1, &sc2, &mc2);
        float d1 = d * (float)sc1;
        float d2 = d * (float)sc2;
        int has_pair_mins = has_block_mins && (mc1 != 0 || mc2 != 0);
        float m1 = 0.0f, m2 = 0.0f;
        if (has_pair_mins) {
            m1 = min_contribution(dmin, mc1);
            m2 = min_contribution(dmin, GO_PLANT == 5 ? mc1 : mc2);
        }
        float qd1, qd2;
        k_chunk_dots(blk, f, c, v + 64 * c, &qd1, &qd2, NULL, NULL);
        float contribution = d1 * qd1 + d2 * qd2;
        if (has_pair_mins) contribution -= m1 * gs[2 * c] + m2 * gs[2 * c + 1];
        part[c] = contribution;
    }
    return part[0] + part[1] + part[2] + part[3];
}

/* Four-way block unrolled row sums shared by dotRowQ4KNoMins
 * (RT/GgufQ4RawDot.java:148-175), dotRowQ4KWithGroupSums (:331-382),
 * dotRowQ5KNoMins (RT/GgufQ5RawDot.java:167-196) and
 * dotRowQ5KWithGroupSums (:393-451). */
static float dot_k_unrolled(const kfmt *f, const uint8_t *row, int64_t cols, const float *x,
                            const float *gs) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int64_t blocks = cols / QK_K, b = 0;
    for (; b + 4 <= blocks; b += 4) {
        for (int u = 0; u < 4; u++) {
            const uint8_t *blk = row + (b + u) * f->bytes;
            const float *v = x + (b + u) * QK_K;
            s[u] += gs ? k_groupsum_block(f, blk, v, gs + (b + u) * 8) : k_nomin_block(f, blk, v);
        }
    }
    float sum = s[0] + s[1] + s[2] + s[3];
    for (; b < blocks; b++) {
        const uint8_t *blk = row + b * f->bytes;
        const float *v = x + b * QK_K;
        sum += gs ? k_groupsum_block(f, blk, v, gs + b * 8) : k_nomin_block(f, blk, v);
    }
    return sum;
}

/* RT/GgufKMeta.java:115-181 (K4_LOW_MIN_MASK / K4_HIGH_MIN_MASK cover every
 * bit that contributes to a 6-bit min code; Q4_K and Q5_K keep dmin and the
 * scale bytes at the same offsets). */
static int k_block_has_mins(const uint8_t *blk) {
    float dmin = go_f16_to_f32(rd16(blk + 2));
    if (dmin == 0.0f) return 0;
    for (int j = 0; j < 8; j++) {
        int sc, m;
        go_k4_scale_min(blk + 4, j, &sc, &m);
        if (m != 0) return 1;
    }
    return 0;
}

static int k_row_has_mins(const kfmt *f, const uint8_t *row, int64_t cols) {
    for (int64_t b = 0; b < cols / QK_K; b++)
        if (k_block_has_mins(row + b * f->bytes)) return 1;
    return 0;
}

static int k_rows_have_mins(const kfmt *f, const uint8_t *data, int64_t row_bytes, int64_t cols,
                            int64_t row_count) {
    for (int64_t r = 0; r < row_count; r++)
        if (k_row_has_mins(f, data + r * row_bytes, cols)) return 1;
    return 0;
}

int go_k_rows_have_mins(int type_id, const uint8_t *data, int64_t row_bytes, int64_t cols,
                        int64_t row_count) {
    if (type_id != GO_Q4_K && type_id != GO_Q5_K) return GO_ERR_UNSUPPORTED;
    return k_rows_have_mins(type_id == GO_Q5_K ? &KF_Q5 : &KF_Q4, data, row_bytes, cols, row_count);
}

int go_q4k_rows_have_mins(const uint8_t *data, int64_t row_bytes, int64_t cols,
                          int64_t row_count) {
    return k_rows_have_mins(&KF_Q4, data, row_bytes, cols, row_count);
}

/* ---- Q6_K raw dots (RT/GgufQ6RawDot.java) -------------------------------- */

/* dotRowQ6KHalf (RT/GgufQ6RawDot.java:402-512) and
 * dotRowQ6KHalfWithGroupSums (:514-629).  lo = ql of this 128-element half,
 * hi = its qh, v = its x, off in {0, 16} picks the 16-element groups
 * off..off+16 of each 32-element quarter.  Without group sums each code
 * enters as (q - 32); with them the codes enter raw and each quarter
 * subtracts 32 x its 16-element x sum, gs[0], gs[2], gs[4], gs[6]. */
static float q6k_half(const uint8_t *lo, const uint8_t *hi, const float *v, int off,
                      float s1, float s2, float s3, float s4, const float *gs) {
    const int bias = gs || GO_PLANT == 2 ? 0 : 32;
    float qd[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int i = off; i < off + 16; i += 8) {
        float t[4] = {0.0f, 0.0f, 0.0f, 0.0f};
        for (int k = 0; k < 8; k++) {
            const int a = lo[i + k], b = lo[32 + i + k], h = hi[i + k];
            const int code[4] = {(a & 0x0F) | ((h & 0x03) << 4),
                                 (b & 0x0F) | (((h >> 2) & 0x03) << 4),
                                 (a >> 4) | (((h >> 4) & 0x03) << 4),
                                 (b >> 4) | (((h >> 6) & 0x03) << 4)};
            for (int j = 0; j < 4; j++) {
                float p = (float)(code[j] - bias) * v[32 * j + i + k];
                t[j] = k ? t[j] + p : p;
            }
        }
        for (int j = 0; j < 4; j++) qd[j] += t[j];
    }
    if (!gs) return s1 * qd[0] + s2 * qd[1] + s3 * qd[2] + s4 * qd[3];
    return s1 * (qd[0] - 32.0f * gs[0]) + s2 * (qd[1] - 32.0f * gs[GO_PLANT == 4 ? 1 : 2]) +
           s3 * (qd[2] - 32.0f * gs[4]) + s4 * (qd[3] - 32.0f * gs[6]);
}

/* dotRowQ6KBlock (RT/GgufQ6RawDot.java:76-132) and dotRowQ6KGroupSumBlock
 * (:334-400): d at byte 208, int8 scales at 192..207; gs (16-element x
 * sums of this block, or NULL) as q6k_half takes them. */
static float q6k_block(const uint8_t *blk, const float *v, const float *gs) {
    const float d = go_f16_to_f32(rd16(blk + 208));
    const int8_t *sc = (const int8_t *)(blk + 192);
    float part[4];
    for (int p = 0; p < 4; p++) {
        const int h = p >> 1, off = 16 * (p & 1);
        const int8_t *s = sc + (GO_PLANT == 3 ? 0 : 8 * h) + (p & 1);
        part[p] = q6k_half(blk + 64 * h, blk + 128 + 32 * h, v + 128 * h, off,
                           d * (float)s[0], d * (float)s[2], d * (float)s[4], d * (float)s[6],
                           gs ? gs + 8 * h + (p & 1) : NULL);
    }
    return part[0] + part[1] + part[2] + part[3];
}

/* dotRowQ6K (RT/GgufQ6RawDot.java:32-74) and dotRowQ6KWithGroupSums
 * (:134-185): four block accumulators, then the tail blocks. */
static float dot_q6_k(const uint8_t *row, int64_t cols, const float *x, const float *gs) {
    float s[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    int64_t blocks = cols / QK_K, b = 0;
    for (; b + 4 <= blocks; b += 4)
        for (int u = 0; u < 4; u++)
            s[u] += q6k_block(row + (b + u) * 210, x + (b + u) * QK_K, gs ? gs + (b + u) * 16 : NULL);
    float sum = s[0] + s[1] + s[2] + s[3];
    for (; b < blocks; b++)
        sum += q6k_block(row + b * 210, x + b * QK_K, gs ? gs + b * 16 : NULL);
    return sum;
}

/* RT/GgufSum.java:30-47, :49-66: per-32 and per-16 sums of x, restated
 * sequentially. */
void go_group_sums32(const float *x, int64_t cols, float *sums) {
    for (int64_t g = 0; g < cols / 32; g++) {
        float s = 0.0f;
        for (int i = 0; i < 32; i++) s += x[32 * g + i];
        sums[g] = s;
    }
}

void go_group_sums16(const float *x, int64_t cols, float *sums) {
    for (int64_t g = 0; g < cols / 16; g++) {
        float s = 0.0f;
        for (int i = 0; i < 16; i++) s += x[16 * g + i];
        sums[g] = s;
    }
}

/* ---- single row dot: RT/GgufRawRoute.java:107-146 ------------------------ */

int go_dot_row(int type_id, const uint8_t *row, int64_t cols, const float *x,
               float *out) {
    int bs = go_block_size(type_id);
    if (bs == 0) return GO_ERR_UNSUPPORTED;
    if (cols % bs != 0) return GO_ERR_ARG;
    if (type_id == GO_Q8_0) {
        *out = dot_q8_0(row, cols, x);
    } else if (type_id == GO_Q4_0) {
        *out = dot_q4_0(row, cols, x);
    } else if (type_id == GO_Q6_K) {
        *out = dot_q6_k(row, cols, x, NULL); /* RT/GgufRawDot.java:146-148 */
    } else {
        /* RT/GgufRawDot.java:78-91 (Q4_K), :120-133 (Q5_K): the row's own
         * min scan picks the inline or the no-min dot. */
        const kfmt *f = type_id == GO_Q5_K ? &KF_Q5 : &KF_Q4;
        *out = k_row_has_mins(f, row, cols) ? dot_k_inline(f, row, cols, x)
                                            : dot_k_unrolled(f, row, cols, x, NULL);
    }
    return GO_OK;
}

/* ---- multi-row mat-vec: RT/GgufRawRoute.java:56-105 and the walkers in
 * RT/GgufQ8RawRows.java:18-41, RT/GgufQ32RawRows.java:18-37,
 * RT/GgufKRawRows.java:122-320, scheduled like RT/GgufParallelConfig.java. */

enum { K_NOMIN = 0, K_DIRECT = 1, K_GROUPSUM = 2 };

typedef struct {
    int type_id;
    const uint8_t *data;
    int64_t cols, row_bytes;
    const float *x;
    const float *group_sums;
    int k_mode;
    float *y;
    int64_t row_begin, row_end;
} go_task;

static void run_rows(const go_task *t) {
    for (int64_t r = t->row_begin; r < t->row_end; r++) {
        const uint8_t *row = t->data + r * t->row_bytes;
        float v;
        if (t->type_id == GO_Q8_0) v = dot_q8_0(row, t->cols, t->x);
        else if (t->type_id == GO_Q4_0) v = dot_q4_0(row, t->cols, t->x);
        else if (t->type_id == GO_Q6_K)
            v = dot_q6_k(row, t->cols, t->x, t->k_mode == K_GROUPSUM ? t->group_sums : NULL);
        else {
            const kfmt *f = t->type_id == GO_Q5_K ? &KF_Q5 : &KF_Q4;
            if (t->k_mode == K_DIRECT) v = dot_k_inline(f, row, t->cols, t->x);
            else v = dot_k_unrolled(f, row, t->cols, t->x,
                                    t->k_mode == K_GROUPSUM ? t->group_sums : NULL);
        }
        t->y[r] = v;
    }
}

typedef struct {
    go_task *tasks;
    int64_t first, count, stride;
} go_worker;

/* Worker w runs chunks w, w + threads, ... in order, the way the ForkJoin
 * common pool spreads 2 x threads chunks over `threads` workers. */
static void *run_worker(void *arg) {
    const go_worker *w = (const go_worker *)arg;
    for (int64_t c = w->first; c < w->count; c += w->stride) run_rows(&w->tasks[c]);
    return NULL;
}

int go_default_threads(void) {
    long n = sysconf(_SC_NPROCESSORS_ONLN);
    return n > 0 ? (int)n : 1;
}

#define GO_MAX_THREADS 512

int go_matvec_rows(int type_id, const uint8_t *data, int64_t rows, int64_t cols,
                   int64_t row_bytes, const float *x, float *y,
                   int64_t row_count, int threads) {
    int bs = go_block_size(type_id);
    if (bs == 0) return GO_ERR_UNSUPPORTED;
    if (cols % bs != 0) return GO_ERR_ARG;
    if (row_count < 0 || row_count > rows) return GO_ERR_ARG;
    if (row_count == 0) return GO_OK;
    if (row_count == 1) return go_dot_row(type_id, data, cols, x, y);

    go_task base;
    memset(&base, 0, sizeof(base));
    base.type_id = type_id;
    base.data = data;
    base.cols = cols;
    base.row_bytes = row_bytes;
    base.x = x;
    base.y = y;
    float *sums = NULL;
    if (type_id == GO_Q4_K || type_id == GO_Q5_K) {
        /* RT/GgufRawMatVec.java:47-79 (Q4_K), :195-267 (Q5_K): tensor-level
         * min scan, then the no-min, direct (2..4 rows) or group-sum walker. */
        const kfmt *f = type_id == GO_Q5_K ? &KF_Q5 : &KF_Q4;
        if (!k_rows_have_mins(f, data, row_bytes, cols, row_count)) {
            base.k_mode = K_NOMIN;
        } else if (row_count <= 4) {
            base.k_mode = K_DIRECT;
        } else {
            base.k_mode = K_GROUPSUM;
            sums = (float *)malloc(sizeof(float) * (size_t)(cols / 32));
            if (!sums) return GO_ERR_ARG;
            go_group_sums32(x, cols, sums);
            base.group_sums = sums;
        }
    } else if (type_id == GO_Q6_K) {
        /* RT/GgufRawMatVec.java:270-296: direct rows for 2..4, else the
         * per-16 x sums and the group-sum walker. */
        if (row_count <= 4) {
            base.k_mode = K_DIRECT;
        } else {
            base.k_mode = K_GROUPSUM;
            sums = (float *)malloc(sizeof(float) * (size_t)(cols / 16));
            if (!sums) return GO_ERR_ARG;
            go_group_sums16(x, cols, sums);
            base.group_sums = sums;
        }
    }

    if (threads <= 0) threads = go_default_threads();
    if (threads > GO_MAX_THREADS) threads = GO_MAX_THREADS;
    int64_t chunks = 0;
    if (threads > 1 && row_count * cols >= 131072) {
        chunks = (int64_t)threads * 2;
        if (chunks > row_count) chunks = row_count;
    }
    if (chunks <= 1) {
        base.row_begin = 0;
        base.row_end = row_count;
        run_rows(&base);
    } else {
        /* RT/GgufParallelConfig.java:63-72: rowsPerChunk + spread remainder. */
        go_task tasks[2 * GO_MAX_THREADS];
        int64_t per = row_count / chunks, extra = row_count % chunks, begin = 0;
        for (int64_t c = 0; c < chunks; c++) {
            int64_t n = per + (c < extra ? 1 : 0);
            tasks[c] = base;
            tasks[c].row_begin = begin;
            tasks[c].row_end = begin + n;
            begin += n;
        }
        go_worker workers[GO_MAX_THREADS];
        pthread_t tids[GO_MAX_THREADS];
        int started[GO_MAX_THREADS];
        int nworkers = threads < chunks ? threads : (int)chunks;
        for (int w = 0; w < nworkers; w++) {
            workers[w].tasks = tasks;
            workers[w].first = w;
            workers[w].count = chunks;
            workers[w].stride = nworkers;
            started[w] = pthread_create(&tids[w], NULL, run_worker, &workers[w]) == 0;
            if (!started[w]) run_worker(&workers[w]);
        }
        for (int w = 0; w < nworkers; w++)
            if (started[w]) pthread_join(tids[w], NULL);
    }
    free(sums);
    return GO_OK;
}

/* ---- MoE router (MoeForwardPass.java:174-203, 286-306) ------------------ */

/* Float.floatToIntBits: one canonical NaN. */
static int32_t float_to_int_bits(float v) {
    int32_t b;
    if (v != v) return 0x7FC00000;
    memcpy(&b, &v, 4);
    return b;
}

/* Float.compare(a, b). */
static int java_float_compare(float a, float b) {
    if (a < b) return -1;
    if (a > b) return 1;
    int32_t ab = float_to_int_bits(a), bb = float_to_int_bits(b);
    return ab == bb ? 0 : (ab < bb ? -1 : 1);
}

/* Math.max(a, b) for floats. */
static float java_max(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == 0.0f && b == 0.0f) return float_to_int_bits(a) == 0 ? a : b;
    return a >= b ? a : b;
}

int go_moe_select_topk(const float *logits, int64_t tokens, int64_t n_experts, int64_t top_k,
                       int sigmoid, int32_t *ids, float *weights) {
    if (tokens < 0 || n_experts <= 0 || top_k <= 0) return GO_ERR_ARG;
    float *p = malloc((size_t)n_experts * sizeof(float));
    int32_t *idx = malloc((size_t)n_experts * sizeof(int32_t));
    if (p == NULL || idx == NULL) {
        free(p);
        free(idx);
        return GO_ERR_ARG;
    }
    for (int64_t t = 0; t < tokens; t++) {
        const float *l = logits + t * n_experts;
        if (sigmoid) { /* :178-181 */
            for (int64_t e = 0; e < n_experts; e++) p[e] = 1.0f / (1.0f + (float)exp((double)(-l[e])));
        } else {       /* :183-196 */
            float max = -INFINITY;
            for (int64_t e = 0; e < n_experts; e++) max = java_max(max, l[e]);
            float sum = 0.0f;
            for (int64_t e = 0; e < n_experts; e++) {
                p[e] = (float)exp((double)(l[e] - max));
                sum += p[e];
            }
            for (int64_t e = 0; e < n_experts; e++) p[e] /= sum;
        }
        /* :288-293: stable sort of the indices, descending Float.compare
         * (insertion sort keeps equal keys in index order, as TimSort does). */
        for (int64_t e = 0; e < n_experts; e++) {
            int64_t j = e;
            while (j > 0 && java_float_compare(p[e], p[idx[j - 1]]) > 0) {
                idx[j] = idx[j - 1];
                j--;
            }
            idx[j] = (int32_t)e;
        }
        /* :295-304 (the arrays start zeroed: ranks past n_experts stay 0). */
        int32_t *oi = ids + t * top_k;
        float *ow = weights + t * top_k;
        for (int64_t k = 0; k < top_k; k++) {
            oi[k] = 0;
            ow[k] = 0.0f;
        }
        float wsum = 0.0f;
        for (int64_t k = 0; k < top_k && k < n_experts; k++) {
            oi[k] = idx[k];
            ow[k] = p[idx[k]];
            wsum += p[idx[k]];
        }
        if (wsum > 0.0f)
            for (int64_t k = 0; k < top_k; k++) ow[k] /= wsum;
    }
    free(p);
    free(idx);
    return GO_OK;
}
