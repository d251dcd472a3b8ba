// gguf_dequant.hip -- bit-exact GGUF row dequantization on gfx950.
//
// Replaces RT/GgufRowDequantizer.dequantizeRow (RT/ = runner/gguf/
// gollek-gguf-core/src/main/java/tech/kayys/gollek/gguf/runtime/) for the
// Q8_0, Q4_0 and Q4_K branches (:97-107, :141-152, :242-252).  Every output
// must equal the Java result bit for bit, so each value is formed with the
// same single IEEE roundings the Java expressions perform and floating-point
// contraction is switched off inside the kernels (no fused multiply-add).
#include "gguf_blocks.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

// One thread per (row, block).  Dequantization is not the bandwidth hot path
// (the GEMV/GEMM kernels decode in registers); it serves dequantizeRow and
// the bit-exact parity contract.
__global__ __launch_bounds__(256) void dequant_q8_0_kernel(const uint8_t *__restrict__ w,
                                                           int64_t row_bytes, int nb,
                                                           int64_t row0, int64_t nrows,
                                                           float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nrows * nb) return;
    const int64_t r = t / nb;
    const int b = (int)(t - r * nb);
    const uint8_t *blk = w + (row0 + r) * row_bytes + (int64_t)b * kQ8BlockBytes;
    const float d = half_bits_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    float *y = out + r * (int64_t)nb * 32 + (int64_t)b * 32;
#pragma unroll
    for (int i = 0; i < 32; i++) y[i] = (float)(int)(int8_t)blk[2 + i] * d;
}

// RT/GgufBlockDequantizer.java:412-413: ((q & 15) - 8) * d + 0.0f; the +0.0f
// turns a -0.0 product into +0.0 and must be kept.
__global__ __launch_bounds__(256) void dequant_q4_0_kernel(const uint8_t *__restrict__ w,
                                                           int64_t row_bytes, int nb,
                                                           int64_t row0, int64_t nrows,
                                                           float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= nrows * nb) return;
    const int64_t r = t / nb;
    const int b = (int)(t - r * nb);
    const uint8_t *blk = w + (row0 + r) * row_bytes + (int64_t)b * kQ4BlockBytes;
    const float d = half_bits_to_float((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
    float *y = out + r * (int64_t)nb * 32 + (int64_t)b * 32;
#pragma unroll
    for (int i = 0; i < 16; i++) {
        const int q = blk[2 + i];
        y[i] = (float)((q & 0x0F) - 8) * d + 0.0f;
        y[16 + i] = (float)((q >> 4) - 8) * d + 0.0f;
    }
}

// RT/GgufKBlockDequantizer.java:31-88.  One thread per (row, superblock,
// 64-element chunk).  dMin == 0 (either sign) takes the no-min branch; a
// zero min code contributes +0.0 even when dMin is NaN or infinite
// (RT/GgufKQuantLayout.java:67-69).
__global__ __launch_bounds__(256) void dequant_q4_k_kernel(const uint8_t *__restrict__ w,
                                                           int64_t row_bytes, int nsb,
                                                           int64_t row0, int64_t nrows,
                                                           float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t per_row = (int64_t)nsb * 4;
    if (t >= nrows * per_row) return;
    const int64_t r = t / per_row;
    const int rem = (int)(t - r * per_row);
    const int s = rem >> 2;
    const int c = rem & 3;
    const uint8_t *blk = w + (row0 + r) * row_bytes + (int64_t)s * kQKBlockBytes;
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
    const uint8_t *q = blk + 16 + 32 * c;
    float *y = out + r * (int64_t)nsb * kQK + (int64_t)s * kQK + 64 * c;
#pragma unroll
    for (int i = 0; i < 32; i++) {
        const int v = q[i];
        y[i] = d1 * (float)(v & 0x0F) - m1;
        y[32 + i] = d2 * (float)(v >> 4) - m2;
    }
}

hipError_t launch_dequant(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                          int64_t row0, int64_t nrows, float *out, hipStream_t stream) {
    if (nrows <= 0) return hipSuccess;
    if (is_k56(type_id)) return launch_dequant_k56(type_id, w, row_bytes, cols, row0, nrows, out, stream);
    const int threads = 256;
    if (type_id == kQ8_0 || type_id == kQ4_0) {
        const int nb = (int)(cols / 32);
        const int64_t total = nrows * nb;
        const unsigned grid = (unsigned)((total + threads - 1) / threads);
        if (type_id == kQ8_0)
            hipLaunchKernelGGL(dequant_q8_0_kernel, dim3(grid), dim3(threads), 0, stream, w,
                               row_bytes, nb, row0, nrows, out);
        else
            hipLaunchKernelGGL(dequant_q4_0_kernel, dim3(grid), dim3(threads), 0, stream, w,
                               row_bytes, nb, row0, nrows, out);
    } else {
        const int nsb = (int)(cols / kQK);
        const int64_t total = nrows * nsb * 4;
        const unsigned grid = (unsigned)((total + threads - 1) / threads);
        hipLaunchKernelGGL(dequant_q4_k_kernel, dim3(grid), dim3(threads), 0, stream, w,
                           row_bytes, nsb, row0, nrows, out);
    }
    return hipGetLastError();
}

}  // namespace gollek
