// gguf_dot4.hpp -- shared device code of the Q4_K integer-dot kernels
// (GEMV in gguf_gemv_dot4.hip, MoE expert FFN in gguf_moe.hip).
//
// A vector x is held as "digit planes": per 32-element group g, a power-of-two
// scale s_g = 2^(e-23) with max|x_g| < 2^e, the exact integers
// X_i = trunc(x_i / s_g) (|X_i| < 2^23) split into three bytes
// X = a' * 2^16 + b' * 2^8 + c' (c', b' unsigned, a' signed), and the fp32
// group sum used by the Q4_K min term.  Nibbles are then contracted with
// v_dot4_u32_u8 / v_dot4_i32_i8 exactly in int32; a group's value is
// s_g * (65536 A + 256 B + C).
#pragma once

#include "gguf_blocks.hpp"

namespace gollek {

constexpr int kDigitWords = 24;  // per 32-element group: 8 c' + 8 b' + 8 a' dwords

__device__ __forceinline__ uint32_t pack_byte(const int *X, int byte) {
    const int sh = 8 * byte;
    return ((uint32_t)(X[0] >> sh) & 0xFFu) | (((uint32_t)(X[1] >> sh) & 0xFFu) << 8) |
           (((uint32_t)(X[2] >> sh) & 0xFFu) << 16) | (((uint32_t)(X[3] >> sh) & 0xFFu) << 24);
}

// Digit planes of x for groups [0, ngroups): four threads per group, eight
// elements each (the quad is always wholly active, so the shuffles are safe).
__device__ inline void build_x_digits(const float *__restrict__ x, int ngroups, uint32_t *dig,
                               float *scl, float *gsum) {
    const int part = threadIdx.x & 3;
    for (int G = threadIdx.x >> 2; G < ngroups; G += blockDim.x >> 2) {
        const float4 *px = reinterpret_cast<const float4 *>(x + 32 * G + 8 * part);
        const float4 a = px[0], b = px[1];
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        float mx = 0.0f, s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            mx = fmaxf(mx, fabsf(v[i]));
            s += v[i];
        }
        mx = fmaxf(mx, __shfl_xor(mx, 1, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 2, 64));
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        int e = 0;
        (void)frexpf(mx, &e);  // mx < 2^e, so |x / 2^(e-23)| < 2^23
        const bool finite = mx <= 3.402823466e38f;
        int X[8];
#pragma unroll
        for (int i = 0; i < 8; i++) X[i] = finite ? (int)ldexpf(v[i], 23 - e) : 0;
        uint2 *out = reinterpret_cast<uint2 *>(dig + kDigitWords * G + 2 * part);
#pragma unroll
        for (int byte = 0; byte < 3; byte++)
            out[4 * byte] = make_uint2(pack_byte(X, byte), pack_byte(X + 4, byte));
        if (part == 0) {
            scl[G] = finite ? ldexpf(1.0f, e - 23) : __builtin_nanf("");
            gsum[G] = s;
        }
    }
}

// One row's contribution from this lane's superblock chunk.
__device__ __forceinline__ float q4k_dot4_row(const uint4 hd, const uint4 qa, const uint4 qb,
                                              const uint32_t (&dg)[2][3][8], const float (&sg)[2],
                                              const float (&xg)[2], int g) {
    const uint32_t wq[8] = {qa.x, qa.y, qa.z, qa.w, qb.x, qb.y, qb.z, qb.w};
    uint32_t c0 = 0, b0 = 0, c1 = 0, b1 = 0;
    int a0 = 0, a1 = 0;
#pragma unroll
    for (int k = 0; k < 8; k++) {
        const uint32_t lo = wq[k] & 0x0F0F0F0Fu;
        const uint32_t hi = (wq[k] >> 4) & 0x0F0F0F0Fu;
        c0 = __builtin_amdgcn_udot4(lo, dg[0][0][k], c0, false);
        b0 = __builtin_amdgcn_udot4(lo, dg[0][1][k], b0, false);
        a0 = __builtin_amdgcn_sdot4((int)lo, (int)dg[0][2][k], a0, false);
        c1 = __builtin_amdgcn_udot4(hi, dg[1][0][k], c1, false);
        b1 = __builtin_amdgcn_udot4(hi, dg[1][1][k], b1, false);
        a1 = __builtin_amdgcn_sdot4((int)hi, (int)dg[1][2][k], a1, false);
    }
    const float s_lo = fmaf((float)a0, 65536.0f, (float)((b0 << 8) + c0));
    const float s_hi = fmaf((float)a1, 65536.0f, (float)((b1 << 8) + c1));

    const float d = half_bits_to_float_fast(hd.x);
    const float dmin = half_bits_to_float_fast(hd.x >> 16);
    uint32_t scp, mnp;
    q4k_pair_codes(hd.y, hd.z, hd.w, g, &scp, &mnp);
    const float p = fmaf((float)(scp >> 8) * sg[1], s_hi, (float)(scp & 0xFFu) * sg[0] * s_lo);
    float mm = fmaf((float)(mnp >> 8), xg[1], (float)(mnp & 0xFFu) * xg[0]);
    // Zero min codes contribute nothing even when dmin is NaN or infinite
    // (RT/GgufQ4RawDot.java:618-634, RT/GgufKQuantLayout.java:67-69).
    mm = mnp ? dmin * mm : 0.0f;
    return fmaf(d, p, -mm);
}

struct RowChunk {
    uint4 h, a, b;  // superblock header, quant bytes 32g..32g+15, 32g+16..32g+31
};

// Loads this lane's chunk of rows r0 + i * RG + rg, i < RB (zero when masked).
template <int RB, int RG>
__device__ __forceinline__ void load_rows(RowChunk (&d)[RB], const uint8_t *__restrict__ w,
                                          int64_t row_bytes, int64_t r0, int64_t row_end, int rg,
                                          int sb, int g, bool act) {
#pragma unroll
    for (int i = 0; i < RB; i++) {
        const int64_t r = r0 + (int64_t)i * RG + rg;
        if (act && r < row_end) {
            const uint8_t *p = w + r * row_bytes + (int64_t)sb * kQKBlockBytes;
            d[i].h = *reinterpret_cast<const uint4 *>(p);
            d[i].a = *reinterpret_cast<const uint4 *>(p + 16 + 32 * g);
            d[i].b = *reinterpret_cast<const uint4 *>(p + 32 + 32 * g);
        } else {
            // Independent zero stores: reading a field back here keeps the
            // whole array in scratch memory.
            d[i].h = make_uint4(0u, 0u, 0u, 0u);
            d[i].a = make_uint4(0u, 0u, 0u, 0u);
            d[i].b = make_uint4(0u, 0u, 0u, 0u);
        }
    }
}


// Per group: 24 digit dwords in LDS, then (after all groups) the scales and
// the group sums.  Bytes of LDS for `ngroups` groups.
__host__ __device__ constexpr size_t digit_lds_bytes(int ngroups) {
    return (size_t)ngroups * (kDigitWords + 2) * sizeof(uint32_t);
}

// This lane's digits for superblock sb, chunk g (groups 8 sb + 2 g and + 1).
__device__ __forceinline__ void load_lane_digits(const uint32_t *dig, const float *scl,
                                                 const float *gsum, int sb, int g, bool act,
                                                 uint32_t (&dg)[2][3][8], float (&sg)[2],
                                                 float (&xg)[2]) {
#pragma unroll
    for (int h = 0; h < 2; h++) {
        sg[h] = 0.0f;
        xg[h] = 0.0f;
#pragma unroll
        for (int p = 0; p < 3; p++)
#pragma unroll
            for (int k = 0; k < 8; k++) dg[h][p][k] = 0u;
    }
    if (!act) return;
    const int G = 8 * sb + 2 * g;
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const uint4 *src = reinterpret_cast<const uint4 *>(dig + kDigitWords * (G + h));
#pragma unroll
        for (int p = 0; p < 3; p++) {
            const uint4 u0 = src[2 * p], u1 = src[2 * p + 1];
            dg[h][p][0] = u0.x; dg[h][p][1] = u0.y; dg[h][p][2] = u0.z; dg[h][p][3] = u0.w;
            dg[h][p][4] = u1.x; dg[h][p][5] = u1.y; dg[h][p][6] = u1.z; dg[h][p][7] = u1.w;
        }
        sg[h] = scl[G + h];
        xg[h] = gsum[G + h];
    }
}

}  // namespace gollek
