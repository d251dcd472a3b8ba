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
#include "gguf_blocks.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

namespace {

constexpr int kDigitWords = 24;  // per 32-element group: 8 c' + 8 b' + 8 a' dwords

__device__ __forceinline__ uint32_t pack_byte(const int *X, int byte) {
    const int sh = 8 * byte;
    return ((uint32_t)(X[0] >> sh) & 0xFFu) | (((uint32_t)(X[1] >> sh) & 0xFFu) << 8) |
           (((uint32_t)(X[2] >> sh) & 0xFFu) << 16) | (((uint32_t)(X[3] >> sh) & 0xFFu) << 24);
}

// Digit planes of x for groups [0, ngroups): four threads per group, eight
// elements each (the quad is always wholly active, so the shuffles are safe).
__device__ void build_x_digits(const float *__restrict__ x, int ngroups, uint32_t *dig,
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

}  // namespace

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
    float sg[2] = {0.0f, 0.0f}, xg[2] = {0.0f, 0.0f};
#pragma unroll
    for (int h = 0; h < 2; h++)
#pragma unroll
        for (int p = 0; p < 3; p++)
#pragma unroll
            for (int k = 0; k < 8; k++) dg[h][p][k] = 0u;
    if (act) {
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
    const size_t lds = (size_t)nsb * 8 * (kDigitWords + 2) * sizeof(uint32_t);
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
