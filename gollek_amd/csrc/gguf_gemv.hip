// gguf_gemv.hip -- fused dequantize-and-multiply GEMV (decode, M = 1) for
// GGUF Q8_0, Q4_0 and Q4_K on gfx950.
//
// Replaces the Java raw mat-vec kernels: RT/GgufQ8RawDot.java:137-184 +
// :783-825 (Q8_0), RT/GgufQ32RawDot.java:33-66 + :427-462 (Q4_0) and
// RT/GgufQ4RawDot.java:331-674 with RT/GgufSum.java:22-46 (Q4_K), where RT/ =
// runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf/runtime/.
// Same value: y[n] = sum_b d_b * (sum_i q_i * x_i) (minus the Q4_K min term
// dmin * m_j * sum_{group j} x); accumulated in fp32 in a different order, so
// parity is within the 1e-3 relative tolerance, not bitwise.
//
// Design (HBM-bound, one pass over the packed weights):
//  * The weights stay in their GGUF byte layout.  A Q4_K superblock (144 B)
//    is 16-byte aligned; pairs of Q8_0 (68 B) and Q4_0 (36 B) blocks are
//    4-byte aligned, so every lane reads whole blocks with wide loads and
//    decodes nibbles / bytes / 6-bit scales in registers.
//  * Each lane owns a fixed slice of the K axis and keeps the matching x
//    values (and their per-group sums for the Q4_K min term) in registers
//    for all the rows its wave visits, so x is read once per wave.
//  * A wave is split into 64/LPR row groups of LPR lanes; a row's partial sums
//    are reduced across its LPR lanes with xor shuffles.
//  * Loads of RB rows are issued before any arithmetic so each wave keeps
//    RB * (bytes per row) in flight.
#include <algorithm>

#include "gguf_block_dot.hpp"
#include "gguf_blocks.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

LaunchTuning &tuning() {
    static LaunchTuning t;
    return t;
}

// ---------------------------------------------------------------- Q4_K ----

__device__ __forceinline__ float q4k_contrib(const uint4 hd, const uint4 q, const float *xl,
                                             const float *xh, float sl, float sh, int g) {
    const float d = half_bits_to_float_fast(hd.x);
    const float dmin = half_bits_to_float_fast(hd.x >> 16);
    uint32_t scp, mnp;
    q4k_pair_codes(hd.y, hd.z, hd.w, g, &scp, &mnp);
    const uint32_t qw[4] = {q.x, q.y, q.z, q.w};
    float al = 0.0f, ah = 0.0f;
#pragma unroll
    for (int k = 0; k < 4; k++) {
        const uint32_t lo = opaque(qw[k] & 0x0F0F0F0Fu);
        const uint32_t hi = opaque(qw[k] & 0xF0F0F0F0u);  // 16 * nibble; 1/16 folded below
#pragma unroll
        for (int b = 0; b < 4; b++) {
            al = fmaf(byte_f(lo, b), xl[4 * k + b], al);
            ah = fmaf(byte_f(hi, b), xh[4 * k + b], ah);
        }
    }
    const float d1 = d * (float)(scp & 0xFFu);
    const float d2 = d * (float)(scp >> 8) * 0.0625f;
    const uint32_t m1 = mnp & 0xFFu, m2 = mnp >> 8;
    // A zero min code contributes nothing even if dmin is NaN or infinite
    // (RT/GgufQ4RawDot.java:618-634, RT/GgufKQuantLayout.java:67-69).
    const float mm1 = m1 ? dmin * (float)m1 : 0.0f;
    const float mm2 = m2 ? dmin * (float)m2 : 0.0f;
    return d1 * al + d2 * ah - (mm1 * sl + mm2 * sh);
}

// Lane gl of a row group handles chunk c = gl & 7 (quant bytes 16c..16c+15)
// of superblocks (gl >> 3) + (LPR / 8) * j, j < ROUNDS.  Chunk c covers
// elements 64g + 16h + [0,16) (low nibbles, sub-block 2g) and
// 64g + 32 + 16h + [0,16) (high nibbles, sub-block 2g+1), g = c/2, h = c%2.
template <int LPR, int ROUNDS, int RB>
__global__ __launch_bounds__(256) void gemv_q4_k_kernel(const uint8_t *__restrict__ w,
                                                        int64_t row_bytes, int nsb,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int64_t rows,
                                                        int64_t rows_per_wave) {
    constexpr int RG = 64 / LPR;
    constexpr int SBS = LPR / 8;
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int rg = lane / LPR;
    const int gl = lane & (LPR - 1);
    const int c = gl & 7, g = c >> 1, h = c & 1, sbl = gl >> 3;

    float xl[ROUNDS][16], xh[ROUNDS][16], sl[ROUNDS], sh[ROUNDS];
    bool act[ROUNDS];
#pragma unroll
    for (int j = 0; j < ROUNDS; j++) {
        const int s = sbl + SBS * j;
        act[j] = s < nsb;
        sl[j] = 0.0f;
        sh[j] = 0.0f;
#pragma unroll
        for (int i = 0; i < 16; i++) {
            xl[j][i] = 0.0f;
            xh[j][i] = 0.0f;
        }
        if (act[j]) {
            const float4 *pl = reinterpret_cast<const float4 *>(x + kQK * s + 64 * g + 16 * h);
            const float4 *ph = reinterpret_cast<const float4 *>(x + kQK * s + 64 * g + 32 + 16 * h);
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const float4 a = pl[k];
                const float4 b = ph[k];
                xl[j][4 * k + 0] = a.x; xl[j][4 * k + 1] = a.y;
                xl[j][4 * k + 2] = a.z; xl[j][4 * k + 3] = a.w;
                xh[j][4 * k + 0] = b.x; xh[j][4 * k + 1] = b.y;
                xh[j][4 * k + 2] = b.z; xh[j][4 * k + 3] = b.w;
            }
#pragma unroll
            for (int i = 0; i < 16; i++) {
                sl[j] += xl[j][i];
                sh[j] += xh[j][i];
            }
        }
    }

    const int64_t row_base = wave * rows_per_wave;
    const int64_t row_end = rows < row_base + rows_per_wave ? rows : row_base + rows_per_wave;
    for (int64_t r0 = row_base; r0 < row_end; r0 += RG * RB) {
        uint4 hd[RB][ROUNDS], qv[RB][ROUNDS];
#pragma unroll
        for (int i = 0; i < RB; i++) {
            const int64_t r = r0 + i * RG + rg;
#pragma unroll
            for (int j = 0; j < ROUNDS; j++) {
                if (r < row_end && act[j]) {
                    const uint8_t *p = w + r * row_bytes + (int64_t)(sbl + SBS * j) * kQKBlockBytes;
                    hd[i][j] = *reinterpret_cast<const uint4 *>(p);
                    qv[i][j] = *reinterpret_cast<const uint4 *>(p + 16 + 16 * c);
                } else {
                    hd[i][j] = make_uint4(0u, 0u, 0u, 0u);
                    qv[i][j] = make_uint4(0u, 0u, 0u, 0u);
                }
            }
        }
        float acc[RB];
#pragma unroll
        for (int i = 0; i < RB; i++) {
            acc[i] = 0.0f;
#pragma unroll
            for (int j = 0; j < ROUNDS; j++)
                acc[i] += q4k_contrib(hd[i][j], qv[i][j], xl[j], xh[j], sl[j], sh[j], g);
            acc[i] = group_sum<LPR>(acc[i]);
        }
        if (gl == 0) {
#pragma unroll
            for (int i = 0; i < RB; i++) {
                const int64_t r = r0 + i * RG + rg;
                if (r < row_end) y[r] = acc[i];
            }
        }
    }
}

// ---------------------------------------------------------------- Q8_0 ----

// Lane gl handles block pair pi = gl + LPR * j: bytes [68 pi, 68 pi + 68) of
// the row = [d0 | q0[32] | d1 | q1[32]], read as 17 aligned dwords.
template <int LPR, int ROUNDS, int RB>
__global__ __launch_bounds__(256) void gemv_q8_0_kernel(const uint8_t *__restrict__ w,
                                                        int64_t row_bytes, int npairs,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int64_t rows,
                                                        int64_t rows_per_wave) {
    constexpr int RG = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int rg = lane / LPR;
    const int gl = lane & (LPR - 1);

    float xv[ROUNDS][64];
    bool act[ROUNDS];
#pragma unroll
    for (int j = 0; j < ROUNDS; j++) {
        const int pi = gl + LPR * j;
        act[j] = pi < npairs;
#pragma unroll
        for (int i = 0; i < 64; i++) xv[j][i] = 0.0f;
        if (act[j]) {
            const float4 *px = reinterpret_cast<const float4 *>(x + 64 * pi);
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const float4 a = px[k];
                xv[j][4 * k + 0] = a.x; xv[j][4 * k + 1] = a.y;
                xv[j][4 * k + 2] = a.z; xv[j][4 * k + 3] = a.w;
            }
        }
    }

    const int64_t row_base = wave * rows_per_wave;
    const int64_t row_end = rows < row_base + rows_per_wave ? rows : row_base + rows_per_wave;
    for (int64_t r0 = row_base; r0 < row_end; r0 += RG * RB) {
        uint32_t v[RB][ROUNDS][17];
#pragma unroll
        for (int i = 0; i < RB; i++) {
            const int64_t r = r0 + i * RG + rg;
#pragma unroll
            for (int j = 0; j < ROUNDS; j++) {
                if (r < row_end && act[j]) {
                    const uint32_t *p = reinterpret_cast<const uint32_t *>(
                        w + r * row_bytes + (int64_t)68 * (gl + LPR * j));
#pragma unroll
                    for (int k = 0; k < 17; k++) v[i][j][k] = p[k];
                } else {
#pragma unroll
                    for (int k = 0; k < 17; k++) v[i][j][k] = 0u;
                }
            }
        }
        float acc[RB];
#pragma unroll
        for (int i = 0; i < RB; i++) {
            acc[i] = 0.0f;
#pragma unroll
            for (int j = 0; j < ROUNDS; j++) {
                const uint32_t *u = v[i][j];
                const float d0 = half_bits_to_float_fast(u[0]);
                const float d1 = half_bits_to_float_fast(u[8] >> 16);
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int e = 0; e < 32; e++) {
                    const int p0 = 2 + e, p1 = 36 + e;
                    s0 = fmaf(sbyte_f(u[p0 >> 2], p0 & 3), xv[j][e], s0);
                    s1 = fmaf(sbyte_f(u[p1 >> 2], p1 & 3), xv[j][32 + e], s1);
                }
                acc[i] += d0 * s0 + d1 * s1;
            }
            acc[i] = group_sum<LPR>(acc[i]);
        }
        if (gl == 0) {
#pragma unroll
            for (int i = 0; i < RB; i++) {
                const int64_t r = r0 + i * RG + rg;
                if (r < row_end) y[r] = acc[i];
            }
        }
    }
}

// ---------------------------------------------------------------- Q4_0 ----

// Lane gl handles block pair pi = gl + LPR * j: bytes [36 pi, 36 pi + 36) =
// [d0 | qs0[16] | d1 | qs1[16]], 9 aligned dwords.  sum (q - 8) x is formed
// as sum q x - 8 sum x with sum x kept per block in registers.
template <int LPR, int ROUNDS, int RB>
__global__ __launch_bounds__(256) void gemv_q4_0_kernel(const uint8_t *__restrict__ w,
                                                        int64_t row_bytes, int npairs,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int64_t rows,
                                                        int64_t rows_per_wave) {
    constexpr int RG = 64 / LPR;
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int rg = lane / LPR;
    const int gl = lane & (LPR - 1);

    float xv[ROUNDS][64], sx[ROUNDS][2];
    bool act[ROUNDS];
#pragma unroll
    for (int j = 0; j < ROUNDS; j++) {
        const int pi = gl + LPR * j;
        act[j] = pi < npairs;
        sx[j][0] = 0.0f;
        sx[j][1] = 0.0f;
#pragma unroll
        for (int i = 0; i < 64; i++) xv[j][i] = 0.0f;
        if (act[j]) {
            const float4 *px = reinterpret_cast<const float4 *>(x + 64 * pi);
#pragma unroll
            for (int k = 0; k < 16; k++) {
                const float4 a = px[k];
                xv[j][4 * k + 0] = a.x; xv[j][4 * k + 1] = a.y;
                xv[j][4 * k + 2] = a.z; xv[j][4 * k + 3] = a.w;
            }
#pragma unroll
            for (int i = 0; i < 32; i++) {
                sx[j][0] += xv[j][i];
                sx[j][1] += xv[j][32 + i];
            }
        }
    }

    const int64_t row_base = wave * rows_per_wave;
    const int64_t row_end = rows < row_base + rows_per_wave ? rows : row_base + rows_per_wave;
    for (int64_t r0 = row_base; r0 < row_end; r0 += RG * RB) {
        uint32_t v[RB][ROUNDS][9];
#pragma unroll
        for (int i = 0; i < RB; i++) {
            const int64_t r = r0 + i * RG + rg;
#pragma unroll
            for (int j = 0; j < ROUNDS; j++) {
                if (r < row_end && act[j]) {
                    const uint32_t *p = reinterpret_cast<const uint32_t *>(
                        w + r * row_bytes + (int64_t)36 * (gl + LPR * j));
#pragma unroll
                    for (int k = 0; k < 9; k++) v[i][j][k] = p[k];
                } else {
#pragma unroll
                    for (int k = 0; k < 9; k++) v[i][j][k] = 0u;
                }
            }
        }
        float acc[RB];
#pragma unroll
        for (int i = 0; i < RB; i++) {
            acc[i] = 0.0f;
#pragma unroll
            for (int j = 0; j < ROUNDS; j++) {
                const uint32_t *u = v[i][j];
                const float d0 = half_bits_to_float_fast(u[0]);
                const float d1 = half_bits_to_float_fast(u[4] >> 16);
                float s[2];
#pragma unroll
                for (int blk = 0; blk < 2; blk++) {
                    const int base = blk ? 20 : 2;  // byte offset of the nibbles
                    const float *xb = xv[j] + 32 * blk;
                    float a = 0.0f;
#pragma unroll
                    for (int e = 0; e < 16; e++) {
                        const int p = base + e;
                        const uint32_t word = u[p >> 2];
                        const float lo = byte_f(opaque(word & 0x0F0F0F0Fu), p & 3);
                        const float hi = byte_f(opaque((word >> 4) & 0x0F0F0F0Fu), p & 3);
                        a = fmaf(lo, xb[e], a);
                        a = fmaf(hi, xb[16 + e], a);
                    }
                    s[blk] = a - 8.0f * sx[j][blk];
                }
                acc[i] += d0 * s[0] + d1 * s[1];
            }
            acc[i] = group_sum<LPR>(acc[i]);
        }
        if (gl == 0) {
#pragma unroll
            for (int i = 0; i < RB; i++) {
                const int64_t r = r0 + i * RG + rg;
                if (r < row_end) y[r] = acc[i];
            }
        }
    }
}

// ------------------------------------------------------------- generic ----

// Any row length and alignment: one wave per row, one lane per block, byte
// loads.  Used for shapes the fast kernels do not cover (odd block counts,
// very long rows, unaligned borrowed buffers: x not 16-byte aligned, or
// weights off the alignment a fast kernel reads them at).
__global__ __launch_bounds__(256) void gemv_generic_kernel(int type_id,
                                                           const uint8_t *__restrict__ w,
                                                           int64_t row_bytes, int nb, int bs,
                                                           int bb, const float *__restrict__ x,
                                                           float *__restrict__ y, int64_t rows) {
    const int lane = threadIdx.x & 63;
    const int64_t r = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    if (r >= rows) return;
    float s = 0.0f;
    for (int b = lane; b < nb; b += 64)
        s += generic_block_dot(type_id, w + r * row_bytes + (int64_t)b * bb, x + (int64_t)b * bs);
    s = group_sum<64>(s);
    if (lane == 0) y[r] = s;
}

// ------------------------------------------------------------ dispatch ----

namespace {

struct GemvPlan {
    int lpr = 0, rounds = 0;  // 0 = generic kernel
};

GemvPlan plan_for(int type_id, int64_t row_bytes, int64_t cols, const void *w, const float *x) {
    GemvPlan p;
    const uintptr_t base = reinterpret_cast<uintptr_t>(w);
    if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) return p;  // float4 loads of x
    if (type_id == kQ4_K) {
        const int64_t nsb = cols / kQK;
        if ((base & 15u) != 0 || (row_bytes & 15) != 0) return p;
        if (nsb % 8 == 0 && nsb <= 32) { p.lpr = 64; p.rounds = (int)(nsb / 8); }
        else if (nsb == 4) { p.lpr = 32; p.rounds = 1; }
        else if (nsb == 2) { p.lpr = 16; p.rounds = 1; }
        else if (nsb == 1 || nsb == 3) { p.lpr = 8; p.rounds = (int)nsb; }
        else if (nsb <= 32) { p.lpr = 64; p.rounds = (int)((nsb + 7) / 8); }
        return p;
    }
    const int64_t nb = cols / 32;
    if (nb % 2 != 0 || (base & 3u) != 0 || (row_bytes & 3) != 0) return p;
    const int64_t npairs = nb / 2;
    if (npairs % 64 == 0 && npairs <= 128) { p.lpr = 64; p.rounds = (int)(npairs / 64); }
    else if (npairs == 32) { p.lpr = 32; p.rounds = 1; }
    else if (npairs == 16) { p.lpr = 16; p.rounds = 1; }
    else if (npairs <= 8) { p.lpr = 8; p.rounds = 1; }
    else if (npairs <= 128) { p.lpr = 64; p.rounds = (int)((npairs + 63) / 64); }
    return p;
}

template <int LPR, int ROUNDS, int RB>
hipError_t launch_fixed(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                        const float *x, float *y, int64_t rows, hipStream_t stream) {
    constexpr int RG = 64 / LPR;
    // About eight waves per CU, each over a run of whole row groups.
    const int64_t target_waves = (int64_t)device_cus() * 8;
    int64_t rpw = (rows + target_waves - 1) / target_waves;
    rpw = ((rpw + RG - 1) / RG) * RG;  // whole row groups
    if (rpw < RG) rpw = RG;
    const int64_t waves = (rows + rpw - 1) / rpw;
    const unsigned grid = (unsigned)((waves + 3) / 4);
    const dim3 block(256);
    if (type_id == kQ4_K)
        hipLaunchKernelGGL((gemv_q4_k_kernel<LPR, ROUNDS, RB>), dim3(grid), block, 0, stream, w,
                           row_bytes, (int)(cols / kQK), x, y, rows, rpw);
    else if (type_id == kQ8_0)
        hipLaunchKernelGGL((gemv_q8_0_kernel<LPR, ROUNDS, RB>), dim3(grid), block, 0, stream, w,
                           row_bytes, (int)(cols / 64), x, y, rows, rpw);
    else
        hipLaunchKernelGGL((gemv_q4_0_kernel<LPR, ROUNDS, RB>), dim3(grid), block, 0, stream, w,
                           row_bytes, (int)(cols / 64), x, y, rows, rpw);
    return hipGetLastError();
}

template <int LPR, int ROUNDS>
hipError_t launch_rb(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                     const float *x, float *y, int64_t rows, hipStream_t stream) {
    const int rb = (type_id == kQ4_K) ? 4 : 2;  // rows per load batch
    if (rb >= 4 && ROUNDS <= 2) return launch_fixed<LPR, ROUNDS, 4>(type_id, w, row_bytes, cols, x, y, rows, stream);
    if (rb >= 2) return launch_fixed<LPR, ROUNDS, 2>(type_id, w, row_bytes, cols, x, y, rows, stream);
    return launch_fixed<LPR, ROUNDS, 1>(type_id, w, row_bytes, cols, x, y, rows, stream);
}

}  // namespace

const char *gemv_variant_name(int type_id, int64_t row_bytes, int64_t cols, const void *w,
                              const float *x) {
    if (q32_mfma_supported(type_id, row_bytes, cols, 1, w, x)) return "gemv_mfma_col_kernel";
    if (type_id == kQ6_K && q6k_mfma_supported(row_bytes, cols, 1, w, x)) return "gemv_q6_k_mfma_tile_kernel";
    if (type_id == kQ5_K && q5k_wide_mfma_supported(row_bytes, cols, 1, w, x)) return "gemv_q4_k_mfma_kernel";
    if (is_k56(type_id))
        return gemv_k56_supported(type_id, row_bytes, w, x) ? "gemv_k56_kernel" : "gemv_generic_kernel";
    const GemvPlan p = plan_for(type_id, row_bytes, cols, w, x);
    if (type_id == kQ4_K && q4k_mfma_supported(row_bytes, cols, 1, w, x)) return "gemv_q4_k_mfma_kernel";
    if (gemv_ring_supported(type_id, row_bytes, cols, 1, w, x)) return "gemv_ring_kernel";
    if (p.lpr == 0) return "gemv_generic_kernel";
    if (type_id == kQ4_K) return "gemv_q4_k_kernel";
    if (type_id == kQ8_0) return "gemv_q8_0_kernel";
    return "gemv_q4_0_kernel";
}

hipError_t launch_gemv(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                       const float *x, float *y, int64_t rows, hipStream_t stream,
                       const uint8_t *prep, int64_t prep_rows) {
    if (rows <= 0) return hipSuccess;
    if (q32_mfma_supported(type_id, row_bytes, cols, rows, w, x))
        return launch_gemv_q32_mfma(type_id, w, row_bytes, cols, x, y, rows, stream, prep, prep_rows);
    if (type_id == kQ6_K && q6k_mfma_supported(row_bytes, cols, rows, w, x))
        return launch_gemv_q6k_mfma(w, row_bytes, cols, x, y, rows, stream);
    if (type_id == kQ5_K && q5k_wide_mfma_supported(row_bytes, cols, rows, w, x))
        return launch_gemv_q5k_wide_mfma(w, row_bytes, cols, x, y, rows, stream);
    if (is_k56(type_id) && gemv_k56_supported(type_id, row_bytes, w, x))
        return launch_gemv_k56(type_id, w, row_bytes, cols, x, y, rows, stream);
    if (type_id == kQ4_K && q4k_mfma_supported(row_bytes, cols, rows, w, x))
        return launch_gemv_q4k_mfma(w, row_bytes, cols, x, y, rows, stream, prep, prep_rows);
    if (gemv_ring_supported(type_id, row_bytes, cols, rows, w, x))
        return launch_gemv_ring(type_id, w, row_bytes, cols, x, y, rows, stream);
    const GemvPlan p = is_k56(type_id) ? GemvPlan() : plan_for(type_id, row_bytes, cols, w, x);
#define GOLLEK_GEMV_CASE(L, R)                                                                \
    if (p.lpr == L && p.rounds == R)                                                          \
        return launch_rb<L, R>(type_id, w, row_bytes, cols, x, y, rows, stream);
    GOLLEK_GEMV_CASE(64, 1)
    GOLLEK_GEMV_CASE(64, 2)
    GOLLEK_GEMV_CASE(64, 3)
    GOLLEK_GEMV_CASE(64, 4)
    GOLLEK_GEMV_CASE(32, 1)
    GOLLEK_GEMV_CASE(16, 1)
    GOLLEK_GEMV_CASE(8, 1)
    GOLLEK_GEMV_CASE(8, 3)
#undef GOLLEK_GEMV_CASE
    const int bs = (type_id == kQ4_K || is_k56(type_id)) ? kQK : 32;
    const int bb = type_id == kQ4_K   ? kQKBlockBytes
                   : type_id == kQ5_K ? 176
                   : type_id == kQ6_K ? 210
                   : type_id == kQ8_0 ? kQ8BlockBytes
                                      : kQ4BlockBytes;
    const int nb = (int)(cols / bs);
    const unsigned grid = (unsigned)((rows + 3) / 4);
    hipLaunchKernelGGL(gemv_generic_kernel, dim3(grid), dim3(256), 0, stream, type_id, w, row_bytes,
                       nb, bs, bb, x, y, rows);
    return hipGetLastError();
}

}  // namespace gollek
