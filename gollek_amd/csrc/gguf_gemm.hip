// gguf_gemm.hip -- Q8_0 x bf16 small-M GEMM (prefill / batched decode) on
// gfx950 bf16 MFMA, fp32 accumulate.
//
// Y[M, N] = X[M, K] . W[N, K]^T with X bf16 and W the GGUF Q8_0 matrix (the
// Linear convention of runner/safetensor/gollek-safetensor-core/src/main/java/
// tech/kayys/gollek/safetensor/core/tensor/AccelOps.java:370-376).  The
// reference has no GGUF GEMM: its prefill runs M independent raw mat-vecs
// (RT/GgufQ8RawDot.java:137-184, RT/ = runner/gguf/gollek-gguf-core/src/main/
// java/tech/kayys/gollek/gguf/runtime/), each y[n] = sum_b d_b * sum_i q_i x_i.
//
// Exactness: the int8 quants are exactly representable in bf16, so each
// v_mfma_f32_16x16x32_bf16 contracts one whole Q8_0 block (K = 32) of X with
// the exact quants in fp32, and the block's fp16 scale d_b is applied to that
// fp32 result before accumulation -- the reference's own block structure.
// Rounding q * d to bf16 instead would cost ~1e-3 relative error per weight.
//
// Tiling: a workgroup of 4 waves owns a BM x BN tile of Y; the waves split it
// WM x WN and, when WK > 1, also split each K stage (the partial tiles are
// summed through LDS at the end).  Each stage moves KB = 64 * WK columns of X
// (bf16) and W (Q8_0 block pairs, 68 aligned bytes, realigned and widened to
// bf16 once per workgroup) into double-buffered LDS; one barrier per stage.
#include "gguf_blocks.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPad = 8;  // bf16 elements of row padding in LDS (bank spread)

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    // Exact: |q| <= 128 is representable in bf16.
    const uint32_t l = __builtin_bit_cast(unsigned short, (__bf16)lo);
    const uint32_t h = __builtin_bit_cast(unsigned short, (__bf16)hi);
    return l | (h << 16);
}

// 4 int8 in a dword -> 2 dwords of bf16 pairs.
__device__ __forceinline__ void i8x4_to_bf16(uint32_t w, uint32_t &a, uint32_t &b) {
    a = pack_bf16x2((float)(int)(int8_t)(w & 0xFFu), (float)(int)(int8_t)((w >> 8) & 0xFFu));
    b = pack_bf16x2((float)(int)(int8_t)((w >> 16) & 0xFFu), (float)(int)(int8_t)(w >> 24));
}

template <int BM, int BN, int KB>
struct Stage {
    uint16_t x[BM][KB + kPad];
    uint16_t w[BN][KB + kPad];
    float d[BN][KB / 32];
};

// Registers holding one stage's global data before it is written to LDS.
template <int XCH, int WIT>
struct StageRegs {
    uint4 x[XCH];
    uint32_t q[WIT][5];
    uint32_t dw[WIT];
};

}  // namespace

template <int BM, int BN, int WM, int WN, int WK>
__global__ __launch_bounds__(256) void gemm_q8_0_bf16_kernel(const uint8_t *__restrict__ W,
                                                             int64_t row_bytes,
                                                             const uint16_t *__restrict__ X,
                                                             float *__restrict__ Y, int M, int N,
                                                             int K) {
    constexpr int KB = 64 * WK;              // K columns per stage
    constexpr int NBLK = KB / 32;            // Q8_0 blocks per row per stage
    constexpr int MT = WM / 16, NT = WN / 16;
    constexpr int WAVES_M = BM / WM, WAVES_N = BN / WN;
    static_assert(WAVES_M * WAVES_N * WK == 4, "four waves per workgroup");
    constexpr int XCHUNKS = BM * KB / 8;     // 16-byte chunks of X per stage
    constexpr int XCH = (XCHUNKS + 255) / 256;
    constexpr int WITEMS = BN * NBLK * 2;    // (row, block, half) items per stage
    constexpr int WIT = (WITEMS + 255) / 256;
    using StageT = Stage<BM, BN, KB>;
    __shared__ StageT st[2];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wk = wave % WK;
    const int wn = (wave / WK) % WAVES_N;
    const int wm = wave / (WK * WAVES_N);
    const int m0 = blockIdx.y * BM;
    const int n0 = blockIdx.x * BN;
    const int nstages = K / KB;

    StageRegs<XCH, WIT> R;

    auto load_global = [&](int s) {
        const int k0 = s * KB;
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + 256 * i;
            const int r = c / (KB / 8), kc = c % (KB / 8);
            R.x[i] = make_uint4(0u, 0u, 0u, 0u);
            if (c < XCHUNKS && m0 + r < M)
                R.x[i] = *reinterpret_cast<const uint4 *>(X + (int64_t)(m0 + r) * K + k0 + 8 * kc);
        }
#pragma unroll
        for (int i = 0; i < WIT; i++) {
            const int it = tid + 256 * i;
            // item -> (row n, block bi, half u): half u holds quants 16u..16u+15
            const int n = it / (NBLK * 2);
            const int rem = it % (NBLK * 2);
            const int bi = rem >> 1, u = rem & 1;
            // Byte offset of block bi inside the row's stage segment; blocks
            // come in 68-byte pairs, so pair starts are 4-byte aligned.
            const int pair = bi >> 1, odd = bi & 1;
            const uint32_t *base = reinterpret_cast<const uint32_t *>(
                W + (int64_t)(n0 + n) * row_bytes + (int64_t)(k0 / 64) * 68 + 68 * pair);
            // Quant bytes of block (pair, odd), half u: odd ? 36 + 16u : 2 + 16u.
            const int first = odd ? 9 + 4 * u : 4 * u;  // first dword covering them
            if (it < WITEMS) {
#pragma unroll
                for (int j = 0; j < 4; j++) R.q[i][j] = base[first + j];
                // even blocks start 2 bytes into a dword and need a fifth one
                R.q[i][4] = odd ? 0u : base[first + 4];
                R.dw[i] = base[odd ? 8 : 0];
            }
        }
    };

    auto store_lds = [&](int buf) {
        StageT &S = st[buf];
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + 256 * i;
            const int r = c / (KB / 8), kc = c % (KB / 8);
            if (c < XCHUNKS) *reinterpret_cast<uint4 *>(&S.x[r][8 * kc]) = R.x[i];
        }
#pragma unroll
        for (int i = 0; i < WIT; i++) {
            const int it = tid + 256 * i;
            if (it >= WITEMS) continue;
            const int n = it / (NBLK * 2);
            const int rem = it % (NBLK * 2);
            const int bi = rem >> 1, u = rem & 1;
            const int odd = bi & 1;
            uint32_t qd[4];
#pragma unroll
            for (int j = 0; j < 4; j++)
                qd[j] = odd ? R.q[i][j] : __builtin_amdgcn_alignbyte(R.q[i][j + 1], R.q[i][j], 2);
            uint32_t o[8];
#pragma unroll
            for (int j = 0; j < 4; j++) i8x4_to_bf16(qd[j], o[2 * j], o[2 * j + 1]);
            uint4 *dst = reinterpret_cast<uint4 *>(&S.w[n][32 * bi + 16 * u]);
            dst[0] = make_uint4(o[0], o[1], o[2], o[3]);
            dst[1] = make_uint4(o[4], o[5], o[6], o[7]);
            if (u == 0) S.d[n][bi] = half_bits_to_float_fast(odd ? (R.dw[i] >> 16) : R.dw[i]);
        }
    };

    f32x4 acc[MT][NT];
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int b = 0; b < NT; b++) acc[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    load_global(0);
    store_lds(0);
    __syncthreads();
    const int lr = lane & 15;       // operand row (A) / column (B) within a 16-tile
    const int lk = 8 * (lane >> 4); // operand k offset within a 32-block
    for (int s = 0; s < nstages; s++) {
        const int buf = s & 1;
        if (s + 1 < nstages) load_global(s + 1);
        const StageT &S = st[buf];
#pragma unroll
        for (int b = 0; b < 2; b++) {
            const int kb = 2 * wk + b;  // block index inside the stage
            bf16x8 A[MT], B[NT];
            float dsc[NT];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                A[mt] = *reinterpret_cast<const bf16x8 *>(&S.x[wm * WM + 16 * mt + lr][32 * kb + lk]);
#pragma unroll
            for (int nt = 0; nt < NT; nt++) {
                B[nt] = *reinterpret_cast<const bf16x8 *>(&S.w[wn * WN + 16 * nt + lr][32 * kb + lk]);
                dsc[nt] = S.d[wn * WN + 16 * nt + lr][kb];
            }
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    const f32x4 t = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                        A[mt], B[nt], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
                    for (int v = 0; v < 4; v++) acc[mt][nt][v] = fmaf(dsc[nt], t[v], acc[mt][nt][v]);
                }
        }
        if (s + 1 < nstages) store_lds(buf ^ 1);
        __syncthreads();
    }

    // D layout of a 16x16 tile: lane holds column lane & 15, rows 4 (lane >> 4) + v.
    if (WK > 1) {
        float *red = reinterpret_cast<float *>(&st[0]);  // stages are free after the loop
        if (wk != 0) {
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        red[(((wave * MT + mt) * NT + nt) * 4 + v) * 64 + lane] = acc[mt][nt][v];
        }
        __syncthreads();
        if (wk != 0) return;
#pragma unroll
        for (int o = 1; o < WK; o++)
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        acc[mt][nt][v] += red[((((wave + o) * MT + mt) * NT + nt) * 4 + v) * 64 + lane];
    }
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = m0 + wm * WM + 16 * mt + 4 * (lane >> 4) + v;
                const int n = n0 + wn * WN + 16 * nt + lr;
                if (m < M) Y[(int64_t)m * N + n] = acc[mt][nt][v];
            }
}

// Any shape: one thread per output, fp32, exact per-block scaling.
__global__ __launch_bounds__(256) void gemm_q8_0_generic_kernel(const uint8_t *__restrict__ W,
                                                                int64_t row_bytes,
                                                                const uint16_t *__restrict__ X,
                                                                float *__restrict__ Y, int M,
                                                                int N, int K) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)M * N) return;
    const int m = (int)(t / N), n = (int)(t % N);
    const uint8_t *row = W + (int64_t)n * row_bytes;
    const uint16_t *xr = X + (int64_t)m * K;
    float acc = 0.0f;
    for (int b = 0; b < K / 32; b++) {
        const uint8_t *blk = row + (int64_t)b * kQ8BlockBytes;
        const float d = half_bits_to_float_fast((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
        float s = 0.0f;
        for (int i = 0; i < 32; i++)
            s = fmaf((float)(int)(int8_t)blk[2 + i], __uint_as_float((uint32_t)xr[32 * b + i] << 16), s);
        acc = fmaf(d, s, acc);
    }
    Y[(int64_t)m * N + n] = acc;
}

namespace {

template <int BM, int BN, int WM, int WN, int WK>
hipError_t launch_tiled(const uint8_t *w, int64_t row_bytes, const uint16_t *x, float *y, int M,
                        int N, int K, hipStream_t stream) {
    const dim3 grid(N / BN, (M + BM - 1) / BM);
    hipLaunchKernelGGL((gemm_q8_0_bf16_kernel<BM, BN, WM, WN, WK>), grid, dim3(256), 0, stream, w,
                       row_bytes, x, y, M, N, K);
    return hipGetLastError();
}

}  // namespace

hipError_t launch_gemm_q8_0_bf16(const uint8_t *w, int64_t row_bytes, const uint16_t *x, float *y,
                                 int M, int N, int K, hipStream_t stream) {
    if (M <= 0) return hipSuccess;
    const bool aligned = (reinterpret_cast<uintptr_t>(w) & 3u) == 0 && (row_bytes & 3) == 0 &&
                         (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    const int v = tuning().gemm_variant;
    if (aligned && v != 1) {
        if (M <= 16 && N % 16 == 0 && K % 256 == 0)
            return launch_tiled<16, 16, 16, 16, 4>(w, row_bytes, x, y, M, N, K, stream);
        if (M <= 128 && N % 16 == 0 && K % 64 == 0)
            return launch_tiled<128, 16, 32, 16, 1>(w, row_bytes, x, y, M, N, K, stream);
        if (N % 64 == 0 && K % 64 == 0)
            return launch_tiled<128, 64, 64, 32, 1>(w, row_bytes, x, y, M, N, K, stream);
    }
    const int64_t total = (int64_t)M * N;
    hipLaunchKernelGGL(gemm_q8_0_generic_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256),
                       0, stream, w, row_bytes, x, y, M, N, K);
    return hipGetLastError();
}

}  // namespace gollek
