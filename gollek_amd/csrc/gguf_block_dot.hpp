// gguf_block_dot.hpp -- one GGUF block (Q8_0 / Q4_0: 32 elements; Q4_K /
// Q5_K / Q6_K: 256) times the matching x values, in fp32 with byte loads:
// any alignment.  The block formulas are the dequantizers' (RT/ =
// runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf/runtime/:
// RT/GgufRowDequantizer.java:141-152 (Q8_0), RT/GgufBlockDequantizer.java:
// 365-414 (Q4_0), RT/GgufKBlockDequantizer.java:31-170, 319-432 (Q4_K, Q5_K,
// Q6_K)) folded into a dot: d * sum(q x), per sub-block scale and min term
// for the K-quants (the min skipped for a zero min code).
#pragma once

#include "gguf_blocks.hpp"

namespace gollek {

__device__ __forceinline__ float generic_block_dot(int type_id, const uint8_t *blk, const float *xb) {
    if (type_id == kQ8_0) {
        const float d = half_bits_to_float_fast((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        float s = 0.0f;
        for (int i = 0; i < 32; i++) s = fmaf((float)(int)(int8_t)blk[2 + i], xb[i], s);
        return d * s;
    }
    if (type_id == kQ4_0) {
        const float d = half_bits_to_float_fast((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        float s = 0.0f;
        for (int i = 0; i < 16; i++) {
            const int q = blk[2 + i];
            s = fmaf((float)((q & 0x0F) - 8), xb[i], s);
            s = fmaf((float)((q >> 4) - 8), xb[16 + i], s);
        }
        return d * s;
    }
    if (type_id == kQ6_K) {  // element e: scale e / 16, code - 32
        const float d = half_bits_to_float_fast((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
        float total = 0.0f;
        for (int g = 0; g < 16; g++) {
            float s = 0.0f;
            for (int k = 0; k < 16; k++) {
                const int e = 16 * g + k, h = e >> 7, j = (e >> 5) & 3, l = e & 31;
                const int ql = blk[64 * h + 32 * (j & 1) + l];
                const int q = ((j < 2 ? ql : ql >> 4) & 0x0F) | (((blk[128 + 32 * h + l] >> (2 * j)) & 3) << 4);
                s = fmaf((float)(q - 32), xb[e], s);
            }
            total = fmaf(d * (float)(int8_t)blk[192 + g], s, total);
        }
        return total;
    }
    // Q4_K, or Q5_K (qh[32] at 16, quants at 48; bit 2c / 2c+1 of qh[i] adds 16)
    const bool q5 = type_id == kQ5_K;
    const int qs = q5 ? 48 : 16;
    const float d = half_bits_to_float_fast((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    const float dmin = half_bits_to_float_fast((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
    float total = 0.0f;
    for (int c = 0; c < 4; c++) {
        int sc1, mc1, sc2, mc2;
        q4k_code(blk + 4, 2 * c, &sc1, &mc1);
        q4k_code(blk + 4, 2 * c + 1, &sc2, &mc2);
        float a1 = 0.0f, a2 = 0.0f, v1 = 0.0f, v2 = 0.0f;
        for (int i = 0; i < 32; i++) {
            const int q = blk[qs + 32 * c + i];
            const int hb = q5 ? blk[16 + i] : 0;
            const float x1 = xb[64 * c + i], x2 = xb[64 * c + 32 + i];
            a1 = fmaf((float)((q & 0x0F) + (((hb >> (2 * c)) & 1) << 4)), x1, a1);
            a2 = fmaf((float)((q >> 4) + (((hb >> (2 * c + 1)) & 1) << 4)), x2, a2);
            v1 += x1;
            v2 += x2;
        }
        const float m1 = mc1 ? dmin * (float)mc1 : 0.0f;
        const float m2 = mc2 ? dmin * (float)mc2 : 0.0f;
        total += d * (float)sc1 * a1 + d * (float)sc2 * a2 - (m1 * v1 + m2 * v2);
    }
    return total;
}


// Elements and bytes of one block of a type (0 for other types).
__host__ __device__ constexpr int block_elems(int type_id) {
    return type_id == kQ8_0 || type_id == kQ4_0 ? 32 : (type_id == kQ4_K || type_id == kQ5_K || type_id == kQ6_K) ? 256 : 0;
}
__host__ __device__ constexpr int block_bytes(int type_id) {
    return type_id == kQ8_0 ? 34 : type_id == kQ4_0 ? 18 : type_id == kQ4_K ? 144 : type_id == kQ5_K ? 176
           : type_id == kQ6_K ? 210 : 0;
}

}  // namespace gollek
