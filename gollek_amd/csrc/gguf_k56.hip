// gguf_k56.hip -- Q5_K and Q6_K: bit-exact row dequantization and the GEMV.
//
// Layouts (256 elements per superblock; RT/ = runner/gguf/gollek-gguf-core/
// src/main/java/tech/kayys/gollek/gguf/runtime/):
//   Q5_K, 176 B: d f16 | dmin f16 | 12 B of 6-bit scale/min codes (as Q4_K)
//                | qh[32] | qs[128].  Chunk c (64 elements) holds
//                q = (qs[32c + i] & 15) + 16 * bit 2c of qh[i] for element
//                64c + i and (qs[32c + i] >> 4) + 16 * bit 2c+1 of qh[i] for
//                64c + 32 + i (RT/GgufKBlockDequantizer.java:91-170).
//   Q6_K, 210 B: ql[128] | qh[64] | int8 scales[16] | d f16.  Half h (128
//                elements) and lane i < 32: ql[64h + i], ql[64h + 32 + i],
//                qh[32h + i] give the four values 128h + {0, 32, 64, 96} + i
//                as 6-bit codes minus 32 with scales[8h + i/16 + {0, 2, 4, 6}]
//                (:319-432).
// Dequantized values round as the Java expressions do: Q5_K
// fl(fl(d1 * q) - m1) with d1 = fl(d * sc) and m1 as for Q4_K (a zero min code,
// or dmin == 0, contributes +0.0); Q6_K fl(fl(d * sc) * (q - 32)).
//
// GEMV: a wave owns a range of rows and walks them R at a time.  Lane l
// takes the 64-element units u = l, l + 64, ... of a row (4 per superblock:
// Q5_K chunk c, Q6_K half h and 16-lane part p); it loads its unit's 64 x
// values once per batch of R rows and the R rows' bytes of that unit
// together, then the row sums are reduced across the wave.  Superblocks
// start at even but not always 4-byte aligned offsets (176 and 210 bytes),
// so 16-byte pieces are read as aligned dwords and realigned with
// v_alignbyte.
#include "gguf_blocks.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

namespace {

constexpr int kQ5KBytes = kQ5KBlockBytes;
constexpr int kQ6KBytes = 210;

__device__ __forceinline__ uint32_t ld_u16(const uint8_t *p) {
    return *reinterpret_cast<const uint16_t *>(p);
}

// The 16 bytes at p (p even).  Reads the aligned dwords covering them; the
// fifth dword only when p is not 4-byte aligned (it then ends 2 bytes past
// the piece: inside the superblock for every Q6_K piece (the last one, the
// scales at 192..207, is followed by d); Q5_K runs only 4-byte aligned).
__device__ __forceinline__ uint4 load16_even(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t *q = reinterpret_cast<const uint32_t *>(a & ~static_cast<uintptr_t>(3));
    const uint32_t v0 = q[0], v1 = q[1], v2 = q[2], v3 = q[3];
    if ((a & 2u) == 0) return make_uint4(v0, v1, v2, v3);
    const uint32_t v4 = q[4];
    return make_uint4(__builtin_amdgcn_alignbyte(v1, v0, 2), __builtin_amdgcn_alignbyte(v2, v1, 2),
                      __builtin_amdgcn_alignbyte(v3, v2, 2), __builtin_amdgcn_alignbyte(v4, v3, 2));
}

// load16_even without a branch, for waves whose lanes mix both alignments:
// always five dword loads, the fifth re-reading the fourth when p is 4-byte
// aligned (so it never leaves the piece), then a shift by p & 3 bytes.
__device__ __forceinline__ uint4 load16_even_uniform(const uint8_t *p) {
    const uintptr_t a = reinterpret_cast<uintptr_t>(p);
    const uint32_t *q = reinterpret_cast<const uint32_t *>(a & ~static_cast<uintptr_t>(3));
    const uint32_t sh = (uint32_t)(a & 3u);
    const uint32_t v0 = q[0], v1 = q[1], v2 = q[2], v3 = q[3], v4 = q[3 + (sh >> 1)];
    return make_uint4(__builtin_amdgcn_alignbyte(v1, v0, sh), __builtin_amdgcn_alignbyte(v2, v1, sh),
                      __builtin_amdgcn_alignbyte(v3, v2, sh), __builtin_amdgcn_alignbyte(v4, v3, sh));
}

// ---- dequantization ----------------------------------------------------------

// One thread per (row, superblock, chunk c): 64 outputs.
__global__ __launch_bounds__(256) void dequant_q5_k_kernel(const uint8_t *__restrict__ w,
                                                           int64_t row_bytes, int nsb, int64_t row0,
                                                           int64_t nrows, float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_row = (int64_t)nsb * 4;
    if (t >= nrows * per_row) return;
    const int64_t r = t / per_row;
    const int rem = (int)(t - r * per_row);
    const int s = rem >> 2, c = rem & 3;
    const uint8_t *blk = w + (row0 + r) * row_bytes + (int64_t)s * kQ5KBytes;
    const float d = half_bits_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    const float dmin = half_bits_to_float((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
    int sc1, mc1, sc2, mc2;
    q4k_code(blk + 4, 2 * c, &sc1, &mc1);
    q4k_code(blk + 4, 2 * c + 1, &sc2, &mc2);
    const float d1 = d * (float)sc1;
    const float d2 = d * (float)sc2;
    float m1 = 0.0f, m2 = 0.0f;
    if (!(dmin == 0.0f)) {
        m1 = mc1 == 0 ? 0.0f : dmin * (float)mc1;
        m2 = mc2 == 0 ? 0.0f : dmin * (float)mc2;
    }
    const uint8_t *qh = blk + 16, *qs = blk + 48 + 32 * c;
    float *y = out + r * (int64_t)nsb * kQK + (int64_t)s * kQK + 64 * c;
#pragma unroll 8
    for (int i = 0; i < 32; i++) {
        const int v = qs[i], hb = qh[i];
        const int lo = (v & 0x0F) + (((hb >> (2 * c)) & 1) << 4);
        const int hi = (v >> 4) + (((hb >> (2 * c + 1)) & 1) << 4);
        y[i] = d1 * (float)lo - m1;
        y[32 + i] = d2 * (float)hi - m2;
    }
}

// One thread per (row, superblock, half h): 128 outputs.
__global__ __launch_bounds__(256) void dequant_q6_k_kernel(const uint8_t *__restrict__ w,
                                                           int64_t row_bytes, int nsb, int64_t row0,
                                                           int64_t nrows, float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_row = (int64_t)nsb * 2;
    if (t >= nrows * per_row) return;
    const int64_t r = t / per_row;
    const int rem = (int)(t - r * per_row);
    const int s = rem >> 1, h = rem & 1;
    const uint8_t *blk = w + (row0 + r) * row_bytes + (int64_t)s * kQ6KBytes;
    const float d = half_bits_to_float((uint32_t)blk[208] | ((uint32_t)blk[209] << 8));
    const uint8_t *ql = blk + 64 * h, *qh = blk + 128 + 32 * h;
    const int8_t *sc = reinterpret_cast<const int8_t *>(blk + 192 + 8 * h);
    float *y = out + r * (int64_t)nsb * kQK + (int64_t)s * kQK + 128 * h;
    for (int half = 0; half < 2; half++) {
        const float s1 = d * (float)sc[half], s2 = d * (float)sc[half + 2];
        const float s3 = d * (float)sc[half + 4], s4 = d * (float)sc[half + 6];
#pragma unroll 4
        for (int i = 16 * half; i < 16 * half + 16; i++) {
            const int a = ql[i], b = ql[32 + i], hb = qh[i];
            y[i] = s1 * (float)(((a & 0x0F) | ((hb & 3) << 4)) - 32);
            y[32 + i] = s2 * (float)(((b & 0x0F) | (((hb >> 2) & 3) << 4)) - 32);
            y[64 + i] = s3 * (float)(((a >> 4) | (((hb >> 4) & 3) << 4)) - 32);
            y[96 + i] = s4 * (float)(((b >> 4) | (((hb >> 6) & 3) << 4)) - 32);
        }
    }
}

// ---- GEMV ------------------------------------------------------------------

// The x values of unit u: element index of x slot k (k < 64).
template <int TYPE>
__device__ __forceinline__ int unit_x_offset(int part, int k) {
    if (TYPE == kQ5_K) return 64 * part + k;              // chunk c = part
    const int h = part >> 1, p = part & 1;                  // Q6_K half, 16-lane part
    return 128 * h + 32 * (k >> 4) + 16 * p + (k & 15);   // groups of 16
}

// Sum over the unit's 64 elements of dequantized weight * x.  xs[g] is the
// sum of the unit's x values of group g (Q5_K: 2 groups of 32, for the min
// terms; Q6_K: 4 groups of 16, for the -32 offset).  Codes are formed four
// at a time in 32-bit words (nibble masks and the high bits shifted into
// bit 4 / bits 4-5 of each byte; no carries cross a byte) and converted with
// v_cvt_f32_ubyteN.
template <int TYPE>
__device__ __forceinline__ float unit_dot(const uint8_t *blk, int part, const float *xv,
                                          const float *xs) {
    if (TYPE == kQ5_K) {
        const int c = part;
        const uint4 hd = load16_even(blk);  // d | dmin | 12 scale bytes
        const float d = half_bits_to_float_fast(hd.x & 0xFFFFu);
        const float dmin = half_bits_to_float_fast(hd.x >> 16);
        uint32_t scp, mnp;
        q4k_pair_codes(hd.y, hd.z, hd.w, c, &scp, &mnp);
        const uint32_t sc1 = scp & 0xFFu, sc2 = scp >> 8, mc1 = mnp & 0xFFu, mc2 = mnp >> 8;
        const uint4 h0 = load16_even(blk + 16);
        const uint4 h1 = load16_even(blk + 32);
        const uint4 q0 = load16_even(blk + 48 + 32 * c);
        const uint4 q1 = load16_even(blk + 64 + 32 * c);
        const uint32_t qw[8] = {q0.x, q0.y, q0.z, q0.w, q1.x, q1.y, q1.z, q1.w};
        const uint32_t hw[8] = {h0.x, h0.y, h0.z, h0.w, h1.x, h1.y, h1.z, h1.w};
        float al = 0.0f, ah = 0.0f;
#pragma unroll
        for (int wi = 0; wi < 8; wi++) {
            const uint32_t lo = opaque((qw[wi] & 0x0F0F0F0Fu) | (((hw[wi] >> (2 * c)) & 0x01010101u) << 4));
            const uint32_t hi =
                opaque(((qw[wi] >> 4) & 0x0F0F0F0Fu) | (((hw[wi] >> (2 * c + 1)) & 0x01010101u) << 4));
#pragma unroll
            for (int b = 0; b < 4; b++) {
                al = fmaf(byte_f(lo, b), xv[4 * wi + b], al);
                ah = fmaf(byte_f(hi, b), xv[32 + 4 * wi + b], ah);
            }
        }
        const bool mins = !(dmin == 0.0f);
        const float m1 = (mins && mc1) ? dmin * (float)mc1 : 0.0f;
        const float m2 = (mins && mc2) ? dmin * (float)mc2 : 0.0f;
        return d * (float)sc1 * al + d * (float)sc2 * ah - (m1 * xs[0] + m2 * xs[1]);
    } else {
        const int h = part >> 1, p = part & 1;
        const uint4 la = load16_even_uniform(blk + 64 * h + 16 * p);
        const uint4 lb = load16_even_uniform(blk + 64 * h + 32 + 16 * p);
        const uint4 hq = load16_even_uniform(blk + 128 + 32 * h + 16 * p);
        const uint4 sv = load16_even_uniform(blk + 192);
        const float d = half_bits_to_float_fast(ld_u16(blk + 208));
        const uint32_t sw0 = h ? sv.z : sv.x, sw1 = h ? sv.w : sv.y;
        const float s1 = (float)(int8_t)(sw0 >> (8 * p)), s2 = (float)(int8_t)(sw0 >> (8 * (2 + p)));
        const float s3 = (float)(int8_t)(sw1 >> (8 * p)), s4 = (float)(int8_t)(sw1 >> (8 * (2 + p)));
        const uint32_t aw[4] = {la.x, la.y, la.z, la.w}, bw[4] = {lb.x, lb.y, lb.z, lb.w};
        const uint32_t hw[4] = {hq.x, hq.y, hq.z, hq.w};
        float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
#pragma unroll
        for (int wi = 0; wi < 4; wi++) {
            const uint32_t A = aw[wi], B = bw[wi], H = hw[wi];
            const uint32_t g0 = opaque((A & 0x0F0F0F0Fu) | ((H & 0x03030303u) << 4));
            const uint32_t g1 = opaque((B & 0x0F0F0F0Fu) | (((H >> 2) & 0x03030303u) << 4));
            const uint32_t g2 = opaque(((A >> 4) & 0x0F0F0F0Fu) | (((H >> 4) & 0x03030303u) << 4));
            const uint32_t g3 = opaque(((B >> 4) & 0x0F0F0F0Fu) | (((H >> 6) & 0x03030303u) << 4));
#pragma unroll
            for (int b = 0; b < 4; b++) {
                a0 = fmaf(byte_f(g0, b), xv[4 * wi + b], a0);
                a1 = fmaf(byte_f(g1, b), xv[16 + 4 * wi + b], a1);
                a2 = fmaf(byte_f(g2, b), xv[32 + 4 * wi + b], a2);
                a3 = fmaf(byte_f(g3, b), xv[48 + 4 * wi + b], a3);
            }
        }
        // sum (q - 32) x = sum q x - 32 sum x per group
        return d * (s1 * (a0 - 32.0f * xs[0]) + s2 * (a1 - 32.0f * xs[1]) +
                    s3 * (a2 - 32.0f * xs[2]) + s4 * (a3 - 32.0f * xs[3]));
    }
}

template <int TYPE, int R>
__global__ __launch_bounds__(256) void gemv_k56_kernel(const uint8_t *__restrict__ w,
                                                       int64_t row_bytes, int nsb,
                                                       const float *__restrict__ x,
                                                       float *__restrict__ y, int64_t rows,
                                                       int64_t rows_per_wave) {
    constexpr int BB = TYPE == kQ5_K ? kQ5KBytes : kQ6KBytes;
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t row_base = wave * rows_per_wave;
    const int64_t row_end = rows < row_base + rows_per_wave ? rows : row_base + rows_per_wave;
    const int units = 4 * nsb;
    for (int64_t r0 = row_base; r0 < row_end; r0 += R) {
        float acc[R];
#pragma unroll
        for (int i = 0; i < R; i++) acc[i] = 0.0f;
        for (int u = lane; u < units; u += 64) {
            const int sb = u >> 2, part = u & 3;
            float xv[64];
#pragma unroll
            for (int k = 0; k < 64; k += 4) {
                const float4 v = *reinterpret_cast<const float4 *>(x + kQK * sb + unit_x_offset<TYPE>(part, k));
                xv[k] = v.x;
                xv[k + 1] = v.y;
                xv[k + 2] = v.z;
                xv[k + 3] = v.w;
            }
            // group sums of x: Q5_K 2 x 32 (slots 0-31, 32-63), Q6_K 4 x 16
            constexpr int NG = TYPE == kQ5_K ? 2 : 4;
            float xs[NG];
#pragma unroll
            for (int g = 0; g < NG; g++) {
                xs[g] = 0.0f;
#pragma unroll
                for (int k = 0; k < 64 / NG; k++) xs[g] += xv[g * (64 / NG) + k];
            }
#pragma unroll
            for (int i = 0; i < R; i++) {
                const int64_t r = r0 + i;
                if (r < row_end)
                    acc[i] += unit_dot<TYPE>(w + r * row_bytes + (int64_t)sb * BB, part, xv, xs);
            }
        }
#pragma unroll
        for (int i = 0; i < R; i++) acc[i] = group_sum<64>(acc[i]);
        if (lane == 0) {
#pragma unroll
            for (int i = 0; i < R; i++)
                if (r0 + i < row_end) y[r0 + i] = acc[i];
        }
    }
}

}  // namespace

bool is_k56(int type_id) { return type_id == kQ5_K || type_id == kQ6_K; }

hipError_t launch_dequant_k56(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                              int64_t row0, int64_t nrows, float *out, hipStream_t stream) {
    if (nrows <= 0) return hipSuccess;
    const int nsb = (int)(cols / kQK);
    const int per = type_id == kQ5_K ? 4 : 2;
    const unsigned grid = (unsigned)((nrows * nsb * per + 255) / 256);
    if (type_id == kQ5_K)
        hipLaunchKernelGGL(dequant_q5_k_kernel, dim3(grid), dim3(256), 0, stream, w, row_bytes, nsb,
                           row0, nrows, out);
    else
        hipLaunchKernelGGL(dequant_q6_k_kernel, dim3(grid), dim3(256), 0, stream, w, row_bytes, nsb,
                           row0, nrows, out);
    return hipGetLastError();
}

// Needs x 16-byte aligned (float4 loads); Q6_K weights 2-byte aligned,
// Q5_K weights 4-byte aligned (its rows are whole 16-byte units, so no piece
// then needs the fifth dword, which for its last piece would lie past the
// superblock).
bool gemv_k56_supported(int type_id, int64_t row_bytes, const void *w, const float *x) {
    const uintptr_t b = reinterpret_cast<uintptr_t>(w);
    if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) return false;
    if (type_id == kQ5_K) return (b & 3u) == 0 && (row_bytes & 3) == 0;
    return (b & 1u) == 0 && (row_bytes & 1) == 0;
}

hipError_t launch_gemv_k56(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                           const float *x, float *y, int64_t rows, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    // Rows per batch R: 4 (x reused over 4 rows) when that still gives the
    // target wave count, else fewer, so small matrices keep enough waves in
    // flight to cover the load latency.
    const int64_t target_waves = (int64_t)device_cus() * 8;
    const int R = rows >= 4 * target_waves ? 4 : (rows >= 2 * target_waves ? 2 : 1);
    int64_t rpw = (rows + target_waves - 1) / target_waves;
    rpw = (rpw + R - 1) / R * R;
    const int64_t waves = (rows + rpw - 1) / rpw;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    const int nsb = (int)(cols / kQK);
#define GOLLEK_K56_LAUNCH(TY, RR)                                                                \
    hipLaunchKernelGGL((gemv_k56_kernel<TY, RR>), dim3(grid), dim3(256), 0, stream, w, row_bytes, \
                       nsb, x, y, rows, rpw)
    if (type_id == kQ5_K) {
        if (R == 4) GOLLEK_K56_LAUNCH(kQ5_K, 4);
        else if (R == 2) GOLLEK_K56_LAUNCH(kQ5_K, 2);
        else GOLLEK_K56_LAUNCH(kQ5_K, 1);
    } else {
        if (R == 4) GOLLEK_K56_LAUNCH(kQ6_K, 4);
        else if (R == 2) GOLLEK_K56_LAUNCH(kQ6_K, 2);
        else GOLLEK_K56_LAUNCH(kQ6_K, 1);
    }
#undef GOLLEK_K56_LAUNCH
    return hipGetLastError();
}

}  // namespace gollek
