// gguf_dot4.hpp -- device code of the Q4_K integer-dot MoE expert passes
// (gguf_moe.hip) and buffer / LDS helpers the matrix-core kernels share.
//
// A vector x is held as "digit planes": per 32-element group g, a power-of-two
// scale s_g = 2^(e-23) with max|x_g| < 2^e, the exact integers
// X_i = rint(x_i / s_g) (|X_i| < 2^23) split into three bytes
// X = a' * 2^16 + b' * 2^8 + c' (c', b' unsigned, a' signed), and the fp32
// group sum used by the Q4_K min term.  Nibbles are then contracted with
// v_dot4_u32_u8 / v_dot4_i32_i8 exactly in int32; a group's value is
// s_g * (65536 A + 256 B + C).
#pragma once

#include "gguf_blocks.hpp"

namespace gollek {

constexpr int kDigitWords = 24;  // per 32-element group: 8 c' + 8 b' + 8 a' dwords

// Nearest integer to v (|v| < 2^23), kept inside the 24-bit two's-complement
// range of the three digit bytes: +-2^23 (a rounding of the largest values)
// becomes +-(2^23 - 1).
__device__ __forceinline__ int round_digits23(float v) {
    const int X = (int)rintf(v);
    return X > 8388607 ? 8388607 : (X < -8388607 ? -8388607 : X);
}

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
        // Maximum of |x| over the bit patterns: NaN and inf order above every
        // finite value, so a non-finite element reaches the branch below
        // (fmaxf would drop a NaN).
        uint32_t mb = 0;
        float s = 0.0f;
#pragma unroll
        for (int i = 0; i < 8; i++) {
            mb = max(mb, __float_as_uint(v[i]) & 0x7FFFFFFFu);
            s += v[i];
        }
        mb = max(mb, (uint32_t)__shfl_xor((int)mb, 1, 64));
        mb = max(mb, (uint32_t)__shfl_xor((int)mb, 2, 64));
        const float mx = __uint_as_float(mb);
        s += __shfl_xor(s, 1, 64);
        s += __shfl_xor(s, 2, 64);
        int e = 0;
        (void)frexpf(mx, &e);  // mx < 2^e, so |x / 2^(e-23)| < 2^23
        const bool finite = mb < 0x7F800000u;
        int X[8];
#pragma unroll
        for (int i = 0; i < 8; i++) X[i] = finite ? round_digits23(ldexpf(v[i], 23 - e)) : 0;
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


// ---- streaming support: buffer descriptors, buffer->LDS row loads --------

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_ptr;

__device__ __forceinline__ uint4 to_uint4(u32x4 v) { return make_uint4(v.x, v.y, v.z, v.w); }

// A 64-bit value the compiler should treat as wave-uniform (it feeds buffer
// descriptors, which live in scalar registers).
__device__ __forceinline__ int64_t wave_uniform(int64_t v) {
    const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)v);
    const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)((uint64_t)v >> 32));
    return (int64_t)(((uint64_t)hi << 32) | lo);
}

// Buffer descriptor over `bytes` bytes at `base` (wave-uniform).  Raw buffer
// loads at offsets at or past `bytes` return zeros without touching memory,
// which is how rows past a wave's range and lanes past a row's end are
// masked without branches (branches would make the load counters
// path-dependent and force a wait for every load before the first use).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t wave_buffer(const uint8_t *base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t *>(base), 0, (int)bytes,
                                             0x00020000);
}

// Offset that is out of range for every descriptor of fewer than 2^31 bytes.
constexpr uint32_t kMaskedOffset = 0x80000000u;

// Cache policy of streamed weight loads: nontemporal (read once per launch,
// so they do not displace x, the digit planes and the outputs).
constexpr int kStreamLoad = 2;

// Copies `row_bytes` bytes at offset `off` of the buffer into the LDS slot
// (NDMA loads of 1 KB: lane l moves bytes 16 l .. 16 l + 15 of each KB; lanes
// past the row read zeros and write them into the slot's padding).  A masked
// row (off == kMaskedOffset) issues the same loads, all out of range, so the
// number of loads in flight is the same on every path.
template <int NDMA>
__device__ __forceinline__ void row_to_lds(__amdgpu_buffer_rsrc_t rs, uint8_t *slot, uint32_t off,
                                           uint32_t row_bytes, int lane) {
#pragma unroll
    for (int k = 0; k < NDMA; k++) {
        const uint32_t in_row = 1024u * k + 16u * lane;
        const uint32_t o = in_row < row_bytes ? off + in_row : kMaskedOffset;
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(slot + 1024 * k), 16, o, 0, 0,
                                                 kStreamLoad);
    }
}

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_mov_dpp(__builtin_bit_cast(int, v), CTRL,
                                                              0xF, 0xF, false));
}

// Sum over the whole wave with DPP (no LDS round trips); valid in lane 63.
__device__ __forceinline__ float wave_sum_to_lane63(float v) {
    v += dpp_f<0xB1>(v);   // quad_perm [1,0,3,2]
    v += dpp_f<0x4E>(v);   // quad_perm [2,3,0,1]
    v += dpp_f<0x124>(v);  // row_ror:4
    v += dpp_f<0x128>(v);  // row_ror:8 -> every lane holds its 16-lane row's sum
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x142,
                                                               0xA, 0xF, false));  // row_bcast:15
    v += __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), 0x143,
                                                               0xC, 0xF, false));  // row_bcast:31
    return v;
}

// Max (of unsigned bit patterns) / sum over aligned groups of eight lanes
// (quad xor 1, xor 2, then the half-row mirror, which pairs lanes 0-3 with
// 7-4 of each eight).
__device__ __forceinline__ uint32_t max8_u32(uint32_t v) {
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0xB1, 0xF, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x4E, 0xF, 0xF, false));
    return max(v, (uint32_t)__builtin_amdgcn_mov_dpp((int)v, 0x141, 0xF, 0xF, false));
}
__device__ __forceinline__ float sum8(float v) {
    v += dpp_f<0xB1>(v);
    v += dpp_f<0x4E>(v);
    return v + dpp_f<0x141>(v);
}

// x digit planes built by eight threads per group, four elements each, in two
// steps so the x loads can be issued before a kernel's weight loads and the
// conversion can run while the weights stream in.  NT = threads of the
// workgroup, XL = float4 loads per thread (8 * ngroups <= XL * NT).
template <int XL>
struct XPart {
    float4 v[XL];
};

template <int NT, int XL>
__device__ __forceinline__ void load_x_parts(XPart<XL> &p, const float *__restrict__ x, int ngroups) {
#pragma unroll
    for (int i = 0; i < XL; i++) {
        // Unconditional load of a clamped index (a branch here would make the
        // compiler wait for the x loads before the weight loads are issued).
        // Threads past the last group hold a copy of its last element; their
        // group index is >= ngroups, so store_x_digits never stores them.
        const int t = threadIdx.x + i * NT;
        p.v[i] = reinterpret_cast<const float4 *>(x)[t < 8 * ngroups ? t : 8 * ngroups - 1];
    }
}

// Every lane of the wave must execute this (the DPP reductions span eight lanes).
template <int NT, int XL>
__device__ __forceinline__ void store_x_digits(const XPart<XL> &p, int ngroups, uint32_t *dig,
                                               float *scl, float *gsum) {
#pragma unroll
    for (int i = 0; i < XL; i++) {
        const int t = threadIdx.x + i * NT;
        const int G = t >> 3, part = t & 7;
        const float v[4] = {p.v[i].x, p.v[i].y, p.v[i].z, p.v[i].w};
        // integer maximum of the |x| bits, so NaN and inf are not dropped
        const uint32_t mb = max8_u32(max(max(__float_as_uint(v[0]) & 0x7FFFFFFFu, __float_as_uint(v[1]) & 0x7FFFFFFFu),
                                         max(__float_as_uint(v[2]) & 0x7FFFFFFFu, __float_as_uint(v[3]) & 0x7FFFFFFFu)));
        const float mx = __uint_as_float(mb);
        const float s = sum8((v[0] + v[1]) + (v[2] + v[3]));
        int e = 0;
        (void)frexpf(mx, &e);  // mx < 2^e, so |x / 2^(e-23)| < 2^23
        const bool finite = mb < 0x7F800000u;
        int X[4];
#pragma unroll
        for (int k = 0; k < 4; k++) X[k] = finite ? round_digits23(ldexpf(v[k], 23 - e)) : 0;
        if (G < ngroups) {
            uint32_t *out = dig + kDigitWords * G + part;
#pragma unroll
            for (int byte = 0; byte < 3; byte++) out[8 * byte] = pack_byte(X, byte);
            if (part == 0) {
                scl[G] = finite ? ldexpf(1.0f, e - 23) : __builtin_nanf("");
                gsum[G] = s;
            }
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
