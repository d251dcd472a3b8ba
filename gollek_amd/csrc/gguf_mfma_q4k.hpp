#pragma once

// gguf_mfma_q4k.hpp -- Q4_K contraction on the gfx950 matrix cores, shared
// by the GEMV (gguf_gemv_mfma.hip) and MoE (gguf_moe_mfma.hip) kernels:
// v_mfma_i32_16x16x64_i8 of 16 weight rows (their nibbles as bytes, the B
// operand) against 64 columns of a vector held as exact integers in
// signed-byte digit planes (the A operand).
//
// A wave that owns one superblock column of 16-row tiles builds its A
// operands (the x digits of that superblock) once, in registers; each tile
// then costs the wave five LDS reads of the 16 rows' header and quant bytes
// of that superblock (B lane n + 16 g: bytes 8 g .. 8 g + 7 of each chunk,
// low nibbles then high nibbles, so A row 4 h + p is zero on the other
// half), four MFMAs and their epilogue.
//
// The vector is held as four balanced signed-byte digit planes of 30-bit integers,
// X_i = trunc(x_i / 2^(e-30)) with max |x| < 2^e over the superblock, so the
// quantisation error of an element is below 2^-30 of that maximum (an fp32
// element has 24 significant bits, so only elements under 2^-6 of the
// maximum lose a fraction at all).  The
// MFMA's A rows 4 h + p (h = sub-block parity, p = plane 0..3) are all live
// for h < 2: lane n + 16 h receives the four plane sums D_p of one (row,
// sub-block), each exact in int32 (|D_p| <= 32 * 15 * 128), and combines
// them as (D2 + 256 D3) 65536 + (D0 + 256 D1) with one fp32 rounding.  The
// sub-block sums of x for the min term are fp32 sums of x itself.

#include "gguf_dot4.hpp"
#include "gguf_kernels.hpp"

namespace gollek {
namespace mfq {

typedef int i32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ int dpp_i(int v) {
    return __builtin_amdgcn_mov_dpp(v, CTRL, 0xF, 0xF, false);
}

// Maximum over the wave (unsigned), returned in every lane.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    v = max(v, (uint32_t)dpp_i<0xB1>((int)v));   // quad_perm [1,0,3,2]
    v = max(v, (uint32_t)dpp_i<0x4E>((int)v));   // quad_perm [2,3,0,1]
    v = max(v, (uint32_t)dpp_i<0x124>((int)v));  // row_ror:4
    v = max(v, (uint32_t)dpp_i<0x128>((int)v));  // row_ror:8
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x142, 0xA, 0xF, false));
    v = max(v, (uint32_t)__builtin_amdgcn_update_dpp(0, (int)v, 0x143, 0xC, 0xF, false));
    return (uint32_t)__builtin_amdgcn_readlane((int)v, 63);
}

// Sum over aligned groups of eight lanes.
__device__ __forceinline__ int sum8_i(int v) {
    v += dpp_i<0xB1>(v);
    v += dpp_i<0x4E>(v);
    return v + dpp_i<0x141>(v);  // row_half_mirror
}


// LDS stores through inline asm, so the compiler does not wait for every
// buffer->LDS load in flight before them.
__device__ __forceinline__ void lds_store_f32(uint32_t addr, float v) {
    asm volatile("ds_write_b32 %0, %1" : : "v"(addr), "v"(v) : "memory");
}

// Reads the 16 rows' header (a_hdr = row n's superblock) and quant bytes
// (a_q = a_hdr + 16 + 8 g) of one tile.
__device__ __forceinline__ void read_tile_superblock(uint32_t a_hdr, uint32_t a_q, u32x4 &hv,
                                                     uint2 (&q)[4]) {
    asm volatile(
        "ds_read_b128 %0, %5\n\t"
        "ds_read_b64 %1, %6\n\t"
        "ds_read_b64 %2, %6 offset:32\n\t"
        "ds_read_b64 %3, %6 offset:64\n\t"
        "ds_read_b64 %4, %6 offset:96\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(hv), "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3])
        : "v"(a_hdr), "v"(a_q)
        : "memory");
}

// Waits until at most N of this wave's loads are outstanding.
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// One 1 KB buffer->LDS load (16 bytes a lane).
__device__ __forceinline__ void col_load(__amdgpu_buffer_rsrc_t rs, uint8_t *dst, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)dst, 16, off, 0, 0, kStreamLoad);
}

// Wave-wide: lane l holds elements 4 l .. 4 l + 3 of a superblock of x.
// Writes the four balanced signed-byte digit planes of X = trunc(x /
// 2^(e-30)), max |x| < 2^e, to `scratch` (1 KB of LDS private to the wave:
// plane p at + 256 p, element i at byte i), leaves this lane's four
// digits of plane p in w[p] and returns the scale 2^(e-30) (NaN when an x
// is not finite).
__device__ __forceinline__ float x_planes4(const float (&v)[4], uint32_t scratch, uint32_t (&w)[4]) {
    const int lane = threadIdx.x & 63;
    uint32_t mb = 0;
#pragma unroll
    for (int k = 0; k < 4; k++) mb = max(mb, __float_as_uint(v[k]) & 0x7FFFFFFFu);
    mb = wave_max_u32(mb);  // NaN and inf order above every finite |x|
    const bool finite = mb < 0x7F800000u;
    int e = 0;
    (void)frexpf(__uint_as_float(mb), &e);  // max |x| < 2^e
    // X = trunc(x / 2^(e-30)), |X| < 2^30 (an fp32 holds 24 significant bits,
    // so only elements below 2^-6 of the maximum lose their fraction: an
    // error under 2^-30 of it).  Adding 0x808080 makes the low three bytes
    // u_p = d_p + 128 of the balanced digits d_p in [-128, 127]; the XOR
    // maps them back to d_p as signed bytes and leaves the top digit
    // d3 = (X + 0x808080) >> 24 in [-64, 64] as byte 3.
    uint32_t Y[4];
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int X = finite ? (int)ldexpf(v[k], 30 - e) : 0;
        Y[k] = ((uint32_t)X + 0x00808080u) ^ 0x00808080u;
    }
    // 4 x 4 byte transpose: w[p] = byte p of Y[0], Y[1], Y[2], Y[3].
    const uint32_t t01l = __builtin_amdgcn_perm(Y[1], Y[0], 0x05010400u);
    const uint32_t t01h = __builtin_amdgcn_perm(Y[1], Y[0], 0x07030602u);
    const uint32_t t23l = __builtin_amdgcn_perm(Y[3], Y[2], 0x05010400u);
    const uint32_t t23h = __builtin_amdgcn_perm(Y[3], Y[2], 0x07030602u);
    w[0] = __builtin_amdgcn_perm(t23l, t01l, 0x05040100u);
    w[1] = __builtin_amdgcn_perm(t23l, t01l, 0x07060302u);
    w[2] = __builtin_amdgcn_perm(t23h, t01h, 0x05040100u);
    w[3] = __builtin_amdgcn_perm(t23h, t01h, 0x07060302u);
    // Plane p at scratch + 256 p; lane l's four elements at byte 4 l.
    asm volatile(
        "ds_write2st64_b32 %0, %1, %2 offset1:1\n\t"
        "ds_write2st64_b32 %0, %3, %4 offset0:2 offset1:3"
        :
        : "v"(scratch + 4 * lane), "v"(w[0]), "v"(w[1]), "v"(w[2]), "v"(w[3])
        : "memory");
    return finite ? ldexpf(1.0f, e - 30) : __builtin_nanf("");
}

// A wave's x operands for one superblock with four digit planes.
struct XOps4 {
    i32x4 A[4];
    float xs4[4], xs;
};

// The same operands held compactly (13 registers instead of 21) by kernels
// that keep several superblocks' operands at once: d[c] = the eight bytes
// of A[c] this lane holds, which x_expand places at A[c] bytes 0..7 (A rows
// m & 7 < 4) or 8..15 (m & 7 >= 4); rows m >= 8 hold zeros, or a second
// vector's operands (x_operands4c<true>).
struct XOpsC {
    uint2 d[4];
    float xs4[4], xs;
};

// Wave-wide: lane l holds elements 4 l .. 4 l + 3 of a superblock of x.
// Writes the digit planes to `scratch` (1 KB of LDS private to the wave),
// reads them back in the A operand layout and leaves the scratch free.
// UPPER: the operands go to A rows 8..15 (m - 8 as m), rows 0..7 are zero
// (a second vector beside the first in one MFMA).
template <bool UPPER = false>
__device__ __forceinline__ void x_operands4c(const float4 xv, uint32_t scratch, XOpsC &o) {
    const int lane = threadIdx.x & 63;
    const float v[4] = {xv.x, xv.y, xv.z, xv.w};
    uint32_t w[4];
    o.xs = x_planes4(v, scratch, w);
    // Sub-block j = lanes 8 j .. 8 j + 7; lane n + 16 g (h = g & 1) needs the
    // sums of sub-blocks 2 c + h.
    const float s8 = sum8((v[0] + v[1]) + (v[2] + v[3]));
    const int h = (lane >> 4) & 1;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const float a = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s8), 16 * c));
        const float b = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, s8), 16 * c + 8));
        o.xs4[c] = h ? b : a;
    }
    // A lane (m, g): plane p = m & 3 of elements 64 c + 8 g .. + 7 (sub-block
    // 2 c) for m < 4, of elements 64 c + 32 + 8 g .. + 7 (2 c + 1) for
    // 4 <= m < 8 (rows m >= 8 read the 4 <= m < 8 bytes and drop them).
    const int m = lane & 15, g = lane >> 4, p = m & 3, ha = (m >> 2) & 1;
    uint2 d[4];
    asm volatile(
        "s_waitcnt lgkmcnt(0)\n\t"
        "ds_read_b64 %0, %4\n\t"
        "ds_read_b64 %1, %4 offset:64\n\t"
        "ds_read_b64 %2, %4 offset:128\n\t"
        "ds_read_b64 %3, %4 offset:192\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(d[0]), "=&v"(d[1]), "=&v"(d[2]), "=&v"(d[3])
        : "v"(scratch + 256 * p + 8 * g + 32 * ha)
        : "memory");
#pragma unroll
    for (int c = 0; c < 4; c++) o.d[c] = (m >= 8) == UPPER ? d[c] : uint2{0u, 0u};
}

__device__ __forceinline__ XOps4 x_expand(const XOpsC &c) {
    const bool lo = (threadIdx.x & 4) == 0;  // rows 0..3 and 8..11: bytes 0..7
    XOps4 o;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const int a = (int)c.d[k].x, b = (int)c.d[k].y;
        o.A[k] = i32x4{lo ? a : 0, lo ? b : 0, lo ? 0 : a, lo ? 0 : b};
        o.xs4[k] = c.xs4[k];
    }
    o.xs = c.xs;
    return o;
}

__device__ __forceinline__ void x_operands4(const float4 xv, uint32_t scratch, XOps4 &o) {
    XOpsC c;
    x_operands4c(xv, scratch, c);
    o = x_expand(c);
}

// One superblock of a 16-row tile with four-plane x: lane n + 16 h returns
// the share of sub-blocks h, 2 + h, 4 + h, 6 + h of row n (lanes 32..63
// return values of the zero A rows, which callers drop).  Q5_K (Q5): qh holds
// the high-bit bytes 8 g .. 8 g + 7 of the lane's elements; bit 2 c (low
// nibbles) or 2 c + 1 (high nibbles) of each becomes bit 4 of the code.
template <bool Q5 = false>
__device__ __forceinline__ float q4k_tile_superblock4(const u32x4 hv, const uint2 (&q)[4],
                                                      const XOps4 &o, const uint2 qh = uint2{0u, 0u}) {
    const int lane = threadIdx.x & 63;
    const int h = (lane >> 4) & 1;
    const i32x4 zero = {0, 0, 0, 0};
    i32x4 D[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        uint32_t b[4] = {q[c].x & 0x0F0F0F0Fu, q[c].y & 0x0F0F0F0Fu, (q[c].x >> 4) & 0x0F0F0F0Fu,
                         (q[c].y >> 4) & 0x0F0F0F0Fu};
        if constexpr (Q5) {
            b[0] |= ((qh.x >> (2 * c)) & 0x01010101u) << 4;
            b[1] |= ((qh.y >> (2 * c)) & 0x01010101u) << 4;
            b[2] |= ((qh.x >> (2 * c + 1)) & 0x01010101u) << 4;
            b[3] |= ((qh.y >> (2 * c + 1)) & 0x01010101u) << 4;
        }
        const i32x4 B = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
        D[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.A[c], B, zero, 0, 0, 0);
    }
    float Sq[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        // |.| < 2^24 for 4-bit codes: exact as a float (one rounding for Q5_K)
        const int lo = D[c][0] + D[c][1] * 256;
        const int hi = D[c][2] + D[c][3] * 256;
        Sq[c] = fmaf((float)hi, 65536.0f, (float)lo);
    }
    const float d = half_bits_to_float_fast(hv.x);
    const float dmin = half_bits_to_float_fast(hv.x >> 16);
    // 6-bit codes (RT/GgufKQuantLayout.java:37-49) of sub-blocks h, 2 + h
    // (bytes 0 and 2 of sc03 / mn03) and 4 + h, 6 + h (of sc47 / mn47)
    const uint32_t hy = hv.y >> (8 * h), hz = hv.z >> (8 * h), hw = hv.w >> (8 * h);
    const uint32_t sc03 = hy & 0x003F003Fu;
    const uint32_t mn03 = hz & 0x003F003Fu;
    const uint32_t sc47 = (hw & 0x000F000Fu) | ((hy >> 2) & 0x00300030u);
    const uint32_t mn47 = ((hw >> 4) & 0x000F000Fu) | ((hz >> 2) & 0x00300030u);
    const float scf[4] = {(float)(sc03 & 0xFFu), (float)((sc03 >> 16) & 0xFFu),
                          (float)(sc47 & 0xFFu), (float)((sc47 >> 16) & 0xFFu)};
    const float mnf[4] = {(float)(mn03 & 0xFFu), (float)((mn03 >> 16) & 0xFFu),
                          (float)(mn47 & 0xFFu), (float)((mn47 >> 16) & 0xFFu)};
    float qs = 0.0f, mm = 0.0f;
    if (__builtin_isfinite(d) && __builtin_isfinite(dmin)) {
#pragma unroll
        for (int c = 0; c < 4; c++) {
            qs = fmaf(scf[c], Sq[c], qs);
            mm = fmaf(mnf[c], o.xs4[c], mm);
        }
        return fmaf(d * o.xs, qs, -(dmin * mm));
    }
    // The reference's products for a non-finite d or dmin: (d sc) per
    // sub-block, and zero min codes skipped even for a NaN or infinite dmin
    // (minContribution, RT/GgufKQuantLayout.java:67-69).
#pragma unroll
    for (int c = 0; c < 4; c++) {
        qs = fmaf(d * scf[c], o.xs * Sq[c], qs);
        mm = fmaf(mnf[c] != 0.0f ? dmin * mnf[c] : 0.0f, o.xs4[c], mm);
    }
    return qs - mm;
}


}  // namespace mfq
}  // namespace gollek
