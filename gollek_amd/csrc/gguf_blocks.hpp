// gguf_blocks.hpp -- GGUF block geometry and device-side decode helpers for
// the CDNA4 (gfx950) kernels.
//
// Block layouts (little endian), as read by the reference Java runtime
// RT/ = runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf/runtime/:
//   Q8_0  34 B : f16 d | int8 q[32]                    y = q * d
//                (RT/GgufRowDequantizer.java:141-152)
//   Q4_0  18 B : f16 d | u8 qs[16]; byte i holds element i (low nibble) and
//                element i+16 (high nibble); y = (nib - 8) * d + 0.0f
//                (RT/GgufBlockDequantizer.java:32-36, :402-414)
//   Q4_K 144 B : f16 d | f16 dmin | u8 scales[12] | u8 qs[128]; chunk c of 32
//                bytes holds elements 64c+i (low) and 64c+32+i (high) of
//                sub-blocks 2c and 2c+1 (RT/GgufKBlockDequantizer.java:31-88)
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace gollek {

enum TypeId : int { kQ4_0 = 2, kQ8_0 = 8, kQ4_K = 12, kQ5_K = 13, kQ6_K = 14 };

constexpr int kQ8BlockBytes = 34;
constexpr int kQ4BlockBytes = 18;
constexpr int kQKBlockBytes = 144;
constexpr int kQ5KBlockBytes = 176;
constexpr int kQK = 256;

// Exact IEEE half -> float, with NaN mapped to the canonical quiet NaN the
// reference's lookup table produces (RT/GgufQuantTables.java:142-164).  Built
// from integer operations so the result does not depend on the shader's
// denormal mode.
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
    const uint32_t sign = (h & 0x8000u) << 16;
    const uint32_t exponent = (h >> 10) & 0x1Fu;
    const uint32_t mantissa = h & 0x3FFu;
    uint32_t bits = sign | ((exponent + 112u) << 23) | (mantissa << 13);
    if (exponent == 0u) {
        // mantissa * 2^-24 is exact and normal in fp32 (or zero).
        const float sub = (float)mantissa * 0x1p-24f;
        bits = __float_as_uint(sub) | sign;
    } else if (exponent == 31u) {
        bits = mantissa ? 0x7FC00000u : (sign | 0x7F800000u);
    }
    return __uint_as_float(bits);
}

// Hardware conversion (v_cvt_f32_f16) for the GEMV/GEMM paths, where outputs
// are compared within a tolerance and a NaN payload cannot matter.
__device__ __forceinline__ float half_bits_to_float_fast(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)(h & 0xFFFFu));
}

// Q4_K 6-bit scale / min codes of sub-blocks 2g and 2g+1, decoded from the
// header dwords hy = scales[0..3], hz = scales[4..7], hw = scales[8..11]
// (RT/GgufKQuantLayout.java:37-49).  For j < 4: sc = b[j] & 63,
// m = b[j+4] & 63; for j >= 4: sc = (b[j+4] & 15) | ((b[j-4] >> 6) << 4),
// m = (b[j+4] >> 4) | ((b[j] >> 6) << 4).  Returns two byte pairs:
// *sc = sc(2g) | sc(2g+1) << 8 and *mn likewise.
__device__ __forceinline__ void q4k_pair_codes(uint32_t hy, uint32_t hz, uint32_t hw, int g,
                                               uint32_t *sc, uint32_t *mn) {
    const int shift = 16 * (g & 1);
    const uint32_t a = (hy >> shift) & 0xFFFFu;
    const uint32_t b = (hz >> shift) & 0xFFFFu;
    const uint32_t c = (hw >> shift) & 0xFFFFu;
    if (g < 2) {
        *sc = a & 0x3F3Fu;
        *mn = b & 0x3F3Fu;
    } else {
        *sc = (c & 0x0F0Fu) | ((a >> 2) & 0x3030u);
        *mn = ((c >> 4) & 0x0F0Fu) | ((b >> 2) & 0x3030u);
    }
}

// Same decode for one code index j in [0, 8) from the 12 scale bytes.
__device__ __forceinline__ void q4k_code(const uint8_t *s, int j, int *sc, int *m) {
    if (j < 4) {
        *sc = s[j] & 63;
        *m = s[j + 4] & 63;
    } else {
        *sc = (s[j + 4] & 0x0F) | ((s[j - 4] >> 6) << 4);
        *m = (s[j + 4] >> 4) | ((s[j] >> 6) << 4);
    }
}

__device__ __forceinline__ float byte_f(uint32_t w, int k) {  // v_cvt_f32_ubyteK
    return (float)((w >> (8 * k)) & 0xFFu);
}

// Hides a value's known bits from the optimiser (emits no instruction).  Used
// on nibble-masked words so that byte_f lowers to one v_cvt_f32_ubyteK per
// element instead of a bit-field extract followed by a conversion.
__device__ __forceinline__ uint32_t opaque(uint32_t v) {
    asm volatile("" : "+v"(v));
    return v;
}

__device__ __forceinline__ float sbyte_f(uint32_t w, int k) {
    return (float)(int)(int8_t)((w >> (8 * k)) & 0xFFu);
}

// Butterfly sum over aligned groups of WIDTH lanes of a wave64.
template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
    for (int o = WIDTH / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
    return v;
}

}  // namespace gollek
