// gguf_gemv_dot4.hip -- Q4_K GEMV (decode, M = 1) on gfx950 with exact
// integer dot products.
//
// Same value as the reference raw Q4_K mat-vec (RT/GgufQ4RawDot.java:331-674
// with RT/GgufSum.java:22-46; RT/ = runner/gguf/gollek-gguf-core/src/main/java/
// tech/kayys/gollek/gguf/runtime/):
//   y[n] = sum_sb sum_j [ d * sc_j * (sum_{i in j} q_i x_i) - dmin * m_j * X_j ]
// with X_j the sum of x over sub-block j.  Tolerance-based parity (1e-3).
//
// Why integers: at 80 % of HBM peak a 4096 x 14336 Q4_K matrix streams in
// ~5 us, which leaves ~170 wave-level VALU instructions per row on 1024 SIMDs.
// Converting every nibble to fp32 and multiplying costs two instructions per
// element (~275 per row in practice) and makes the kernel VALU-bound.  Here
// each 32-element group of x is written exactly as X_i = trunc(x_i / s_g) with
// a power-of-two scale s_g and |X_i| < 2^23, split into three bytes
// X = a' * 2^16 + b' * 2^8 + c' (c', b' unsigned, a' signed), and the nibbles
// are contracted with v_dot4_u32_u8 / v_dot4_i32_i8: 4 MACs per instruction,
// exact in int32.  A group's fp32 value is s_g * (65536 A + 256 B + C), so the
// per-element error is at most s_g (2^-23 of the group's max |x|), the same
// order as fp32 accumulation.
//
// Layout: 4 lanes cover one 144-byte superblock; lane g of the four reads the
// 16-byte header and the 32 quant bytes of chunk g (elements 64g..64g+31 in
// the low nibbles, 64g+32..64g+63 in the high nibbles) -- three 16-byte loads.
// A wave splits into 64/LPR row groups of LPR = 4 * superblocks-per-row
// lanes.  The first batch of weight loads is issued before the workgroup
// converts x into digit planes in LDS, so the HBM stream starts at once.
#include "gguf_dot4.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

// One batch of RB rows per row group: reduce across the LPR lanes and store.
template <int LPR, int RB>
__device__ __forceinline__ void finish_rows(const RowChunk (&d)[RB], const uint32_t (&dg)[2][3][8],
                                            const float (&sg)[2], const float (&xg)[2], int g,
                                            int gl, int rg, int64_t r0, int64_t row_end,
                                            float *__restrict__ y) {
    constexpr int RG = 64 / LPR;
    float acc[RB];
#pragma unroll
    for (int i = 0; i < RB; i++) {
        acc[i] = q4k_dot4_row(d[i].h, d[i].a, d[i].b, dg, sg, xg, g);
        acc[i] = group_sum<LPR>(acc[i]);
    }
    if (gl == 0) {
#pragma unroll
        for (int i = 0; i < RB; i++) {
            const int64_t r = r0 + (int64_t)i * RG + rg;
            if (r < row_end) y[r] = acc[i];
        }
    }
}

// SINGLE: every row of the wave fits one batch (rows_per_wave <= RB * 64/LPR),
// so all of the wave's weight loads are in flight before anything else runs.
// Otherwise two batches ping-pong: one is loading while the other computes.
template <int LPR, int RB, bool SINGLE>
__global__ __launch_bounds__(512) void gemv_q4_k_dot4_kernel(const uint8_t *__restrict__ w,
                                                             int64_t row_bytes, int nsb,
                                                             const float *__restrict__ x,
                                                             float *__restrict__ y, int64_t rows,
                                                             int64_t rows_per_wave) {
    extern __shared__ uint32_t smem[];
    constexpr int RG = 64 / LPR;
    constexpr int STEP = RG * RB;
    const int ngroups = nsb * 8;
    uint32_t *dig = smem;
    float *scl = reinterpret_cast<float *>(smem + kDigitWords * ngroups);
    float *gsum = scl + ngroups;

    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int rg = lane / LPR;
    const int gl = lane & (LPR - 1);
    const int g = gl & 3;
    const int sb = gl >> 2;
    const bool act = sb < nsb;
    const int64_t row_base = wave * rows_per_wave;
    const int64_t row_end = rows < row_base + rows_per_wave ? rows : row_base + rows_per_wave;

    RowChunk A[RB];
    load_rows<RB, RG>(A, w, row_bytes, row_base, row_end, rg, sb, g, act);

    build_x_digits(x, ngroups, dig, scl, gsum);
    __syncthreads();

    uint32_t dg[2][3][8];
    float sg[2], xg[2];
    load_lane_digits(dig, scl, gsum, sb, g, act, dg, sg, xg);

    if (SINGLE) {
        finish_rows<LPR, RB>(A, dg, sg, xg, g, gl, rg, row_base, row_end, y);
        return;
    }
    for (int64_t r0 = row_base; r0 < row_end; r0 += 2 * STEP) {
        RowChunk B[RB];
        load_rows<RB, RG>(B, w, row_bytes, r0 + STEP, row_end, rg, sb, g, act);
        finish_rows<LPR, RB>(A, dg, sg, xg, g, gl, rg, r0, row_end, y);
        load_rows<RB, RG>(A, w, row_bytes, r0 + 2 * STEP, row_end, rg, sb, g, act);
        if (r0 + STEP < row_end) finish_rows<LPR, RB>(B, dg, sg, xg, g, gl, rg, r0 + STEP, row_end, y);
    }
}

namespace {

constexpr int kDot4Threads = 512;

template <int LPR, int RB>
hipError_t launch_dot4(const uint8_t *w, int64_t row_bytes, int nsb, const float *x, float *y,
                       int64_t rows, int64_t rpw, hipStream_t stream) {
    constexpr int RG = 64 / LPR;
    const int64_t waves = (rows + rpw - 1) / rpw;
    const int waves_per_block = kDot4Threads / 64;
    const unsigned grid = (unsigned)((waves + waves_per_block - 1) / waves_per_block);
    const size_t lds = digit_lds_bytes(nsb * 8);
    if (rpw <= (int64_t)RG * RB)
        hipLaunchKernelGGL((gemv_q4_k_dot4_kernel<LPR, RB, true>), dim3(grid), dim3(kDot4Threads),
                           lds, stream, w, row_bytes, nsb, x, y, rows, rpw);
    else
        hipLaunchKernelGGL((gemv_q4_k_dot4_kernel<LPR, RB, false>), dim3(grid), dim3(kDot4Threads),
                           lds, stream, w, row_bytes, nsb, x, y, rows, rpw);
    return hipGetLastError();
}

// Rows per wave: enough waves to fill every CU with `waves_per_cu` of them,
// whole row groups; a single batch when that covers the wave's rows.
template <int LPR>
hipError_t launch_dot4_auto(const uint8_t *w, int64_t row_bytes, int nsb, const float *x,
                            float *y, int64_t rows, hipStream_t stream) {
    constexpr int RG = 64 / LPR;
    const LaunchTuning &t = tuning();
    int64_t rpw = t.gemv_rows_per_wave;
    if (rpw <= 0) {
        const int64_t target_waves = (int64_t)t.cu_count * t.gemv_waves_per_cu;
        rpw = (rows + target_waves - 1) / target_waves;
    }
    rpw = ((rpw + RG - 1) / RG) * RG;
    if (rpw < RG) rpw = RG;
    // Measured on MI355X (4096 x 14336 and 4096 x 128256): two-row ping-pong
    // batches beat one eight-row batch, whose 165 VGPRs cost occupancy.
    const int rb = t.gemv_row_batch;
    if (rb == 8 && rpw <= (int64_t)RG * 8)
        return launch_dot4<LPR, 8>(w, row_bytes, nsb, x, y, rows, rpw, stream);
    if (rb == 4) return launch_dot4<LPR, 4>(w, row_bytes, nsb, x, y, rows, rpw, stream);
    return launch_dot4<LPR, 2>(w, row_bytes, nsb, x, y, rows, rpw, stream);
}

}  // namespace

bool q4k_dot4_supported(int64_t row_bytes, int64_t cols, const void *w, const float *x) {
    if (tuning().gemv_variant == 1) return false;  // forced fp32 path
    const int64_t nsb = cols / kQK;
    return nsb >= 1 && nsb <= 16 && (reinterpret_cast<uintptr_t>(w) & 15u) == 0 &&
           (row_bytes & 15) == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

hipError_t launch_gemv_q4k_dot4(const uint8_t *w, int64_t row_bytes, int64_t cols,
                                const float *x, float *y, int64_t rows, hipStream_t stream) {
    const int nsb = (int)(cols / kQK);
    if (nsb > 8) return launch_dot4_auto<64>(w, row_bytes, nsb, x, y, rows, stream);
    if (nsb > 4) return launch_dot4_auto<32>(w, row_bytes, nsb, x, y, rows, stream);
    if (nsb > 2) return launch_dot4_auto<16>(w, row_bytes, nsb, x, y, rows, stream);
    if (nsb > 1) return launch_dot4_auto<8>(w, row_bytes, nsb, x, y, rows, stream);
    return launch_dot4_auto<4>(w, row_bytes, nsb, x, y, rows, stream);
}

}  // namespace gollek
