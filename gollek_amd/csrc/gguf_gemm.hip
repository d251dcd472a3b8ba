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
// Two kernels.  M >= 256: gemm_q8_0_bf16_big_kernel (128 x 64 workgroup
// tiles, register-pipelined global loads, described below).  Smaller M:
// gemm_q8_0_bf16_kernel, where a workgroup of 4 waves owns a BM x BN tile of
// Y; the waves split it WM x WN and, when WK > 1, also split each K stage
// (the partial tiles are summed through LDS at the end).  Each stage moves
// KB = 64 * WK columns of X (bf16) and W (Q8_0 block pairs, 68 aligned bytes,
// realigned and widened to bf16 once per workgroup) into double-buffered LDS;
// one barrier per stage.
#include "gguf_blocks.hpp"
#include "gguf_dot4.hpp"
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

// ---- large-M kernel -----------------------------------------------------------
//
// Workgroup tile 128 (M) x 64 (N), four waves of 64 x 32 (2 x 2), K in stages
// of one Q8_0 block pair (64 columns).  Operands are staged in LDS as bf16
// (X as stored, W converted once per workgroup: each int8 quant becomes an
// exact bf16, each fp16 block scale an fp32), in 128-byte rows whose 16-byte
// chunks are XOR-swizzled by row so the MFMA fragment reads are free of bank
// conflicts.  Global loads run kPipe stages ahead in registers (raw buffer
// loads: rows past M read zeros); one barrier per stage with two LDS buffers.
// Per Q8_0 block every 16 x 16 output tile takes one v_mfma_f32_16x16x32_bf16
// with a zero accumulator and the fp32 scale is applied with four FMAs.
// Workgroups map to tiles so that each XCD's workgroups share M tiles: X,
// re-read by every N tile, then comes from that XCD's L2.

namespace {

constexpr int kBigBM = 128, kBigBN = 64;

// Byte offset of bf16 chunk kc (8 elements) of row r in a tile of 128-byte
// rows whose 16-byte chunks are XOR-swizzled by row pair, so the 16-byte
// fragment reads of 16 consecutive rows fall in distinct banks.
constexpr int kRowStride = 128;
__device__ __forceinline__ uint32_t swz(int r, int kc) {
    return (uint32_t)(r * kRowStride + 16 * (kc ^ ((r >> 1) & 7)));
}

template <int XCH>
struct BigRegs {
    u32x4 x[XCH];  // 16-byte chunks of X
    u32x4 q;       // W quant dwords
    uint32_t q5;   // fifth quant dword (even block) or the scale dword (odd block)
};

struct BigStage {
    uint8_t x[kBigBM * kRowStride];
    uint8_t w[kBigBN * kRowStride];
    float d[kBigBN][4];  // [.][b] block scales; [.][2 + b] unused (see stash)
};

}  // namespace

template <int kPipe, int WAVES_M, int WAVES_N>
__global__ __launch_bounds__(64 * WAVES_M * WAVES_N) void gemm_q8_0_bf16_big_kernel(
    const uint8_t *__restrict__ W, int64_t row_bytes, const uint16_t *__restrict__ X,
    float *__restrict__ Y, int M, int N, int K) {
    constexpr int NTH = 64 * WAVES_M * WAVES_N;
    constexpr int WM = kBigBM / WAVES_M, WN = kBigBN / WAVES_N;
    constexpr int MT = WM / 16, NT = WN / 16;
    constexpr int XCH = kBigBM * 8 / NTH;   // X chunks per thread per stage
    constexpr int WIT = kBigBN * 4;          // W (row, block, half) items per stage
    static_assert(XCH * NTH == kBigBM * 8 && WIT <= NTH && NTH % WIT == 0, "staging split");
    __shared__ __attribute__((aligned(16))) BigStage st[2];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int n_tiles = N / kBigBN;
    // Tiles in M-major order t = m * n_tiles + n.  Workgroups are dealt to the
    // eight XCDs round robin (blockIdx % 8), so when the grid divides by 8,
    // XCD j takes the contiguous tiles [j G/8, (j+1) G/8): its workgroups share
    // one or two M tiles and the X rows they read stay in that XCD's L2.
    const int G = (int)gridDim.x;
    const int t = (G % 8 == 0) ? (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int mt_idx = t / n_tiles, nt_idx = t % n_tiles;
    const int m0 = mt_idx * kBigBM, n0 = nt_idx * kBigBN;
    const int nst = K / 64;

    // X rows m0.. (zeros past M), W rows n0.. (N % 64 == 0 by dispatch).
    const __amdgpu_buffer_rsrc_t xs = wave_buffer(
        reinterpret_cast<const uint8_t *>(X) + (int64_t)m0 * K * 2,
        (uint32_t)((int64_t)(M - m0 < kBigBM ? M - m0 : kBigBM) * K * 2));
    const __amdgpu_buffer_rsrc_t ws =
        wave_buffer(W + (int64_t)n0 * row_bytes, (uint32_t)(kBigBN * row_bytes));

    // Staging roles.  X: chunks c = tid + NTH i (row c / 8, chunk c % 8).
    // W: item tid % WIT: row, block (0/1) and 16-quant half of the pair; with
    // more threads than items the spares repeat an item (same loads, same
    // values to the same LDS bytes), which keeps the code free of branches.
    const int wit = tid % WIT;
    const int wr = wit >> 2, wb = (wit >> 1) & 1, wu = wit & 1;
    const uint32_t w_q = (uint32_t)(wr * row_bytes) + (wb ? 36u + 16u * wu : 16u * wu);
    const uint32_t w_5 = (uint32_t)(wr * row_bytes) + (wb ? 32u : 16u * wu + 16u);

    // Loads of stage s; stages past the end read zeros (masked offsets), so
    // every pipeline step issues the same loads and the load counters stay
    // exact (a conditional load would make the compiler wait for all of them).
    auto load = [&](BigRegs<XCH> &R, int s) {
        const bool live = s < nst;
        const uint32_t k0b = (uint32_t)s * 128u;  // bf16 bytes
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + NTH * i;
            const uint32_t o = (uint32_t)((c >> 3) * K * 2) + k0b + 16u * (c & 7);
            R.x[i] = __builtin_amdgcn_raw_buffer_load_b128(xs, live ? o : kMaskedOffset, 0, 0);
        }
        const uint32_t pb = (uint32_t)s * 68u;
        R.q = __builtin_amdgcn_raw_buffer_load_b128(ws, live ? w_q + pb : kMaskedOffset, 0, 0);
        R.q5 = __builtin_amdgcn_raw_buffer_load_b32(ws, live ? w_5 + pb : kMaskedOffset, 0, 0);
    };
    auto stash = [&](const BigRegs<XCH> &R, BigStage &S) {
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int c = tid + NTH * i;
            *reinterpret_cast<u32x4 *>(S.x + swz(c >> 3, c & 7)) = R.x[i];
        }
        // Even blocks: the quants start 2 bytes into the first dword.
        const int sh = wb ? 0 : 2;
        uint32_t qd[4];
        qd[0] = __builtin_amdgcn_alignbyte(R.q.y, R.q.x, sh);
        qd[1] = __builtin_amdgcn_alignbyte(R.q.z, R.q.y, sh);
        qd[2] = __builtin_amdgcn_alignbyte(R.q.w, R.q.z, sh);
        qd[3] = __builtin_amdgcn_alignbyte(R.q5, R.q.w, sh);
        uint32_t o[8];
#pragma unroll
        for (int j = 0; j < 4; j++) i8x4_to_bf16(qd[j], o[2 * j], o[2 * j + 1]);
        const int kc = 4 * wb + 2 * wu;
        *reinterpret_cast<u32x4 *>(S.w + swz(wr, kc)) = u32x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<u32x4 *>(S.w + swz(wr, kc + 1)) = u32x4{o[4], o[5], o[6], o[7]};
        // Only the first half of an even block holds its scale; the second half
        // stores into a slot nobody reads (d[.][2 + b]) instead of branching.
        S.d[wr][wb + 2 * wu] = half_bits_to_float_fast(wb ? (R.q5 >> 16) : R.q.x);
    };

    f32x4 acc[MT][NT];
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int b = 0; b < NT; b++) acc[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

    // Pipeline: registers hold stages s + 1 .. s + kPipe; LDS buffer s & 1
    // holds stage s.  In stage s a wave issues its MFMAs, then converts and
    // writes stage s + 1 into the other buffer while they run, applies the
    // scales, and meets the others at the one barrier of the stage.
    // The host guarantees nst % kPipe == 0 and nst >= kPipe, so the steady
    // state below has no branches around loads.
    BigRegs<XCH> R[kPipe];
#pragma unroll
    for (int j = 0; j < kPipe; j++) load(R[j], j);
    stash(R[0], st[0]);
    load(R[0], kPipe);
    __syncthreads();

    const int lr = lane & 15, lk = lane >> 4;
    for (int s0 = 0; s0 < nst; s0 += kPipe) {
#pragma unroll
        for (int j = 0; j < kPipe; j++) {
            const int s = s0 + j;
            const BigStage &S = st[s & 1];
            f32x4 part[2][MT][NT];
            float dsc[2][NT];
#pragma unroll
            for (int kb = 0; kb < 2; kb++) {
                bf16x8 A[MT], B[NT];
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    A[mt] = *reinterpret_cast<const bf16x8 *>(S.x + swz(wm * WM + mt * 16 + lr, 4 * kb + lk));
#pragma unroll
                for (int nt = 0; nt < NT; nt++) {
                    B[nt] = *reinterpret_cast<const bf16x8 *>(S.w + swz(wn * WN + nt * 16 + lr, 4 * kb + lk));
                    dsc[kb][nt] = S.d[wn * WN + nt * 16 + lr][kb];
                }
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int nt = 0; nt < NT; nt++)
                        part[kb][mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
                            A[mt], B[nt], f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            }
            // Stage s + 1 sits in R[(j + 1) % kPipe]: write it to the other
            // buffer while the MFMAs run (past the last stage this writes
            // zeros nobody reads), then refill the slot with s + 1 + kPipe.
            BigRegs<XCH> &Rn = R[(j + 1) % kPipe];
            stash(Rn, st[(s + 1) & 1]);
            load(Rn, s + 1 + kPipe);
#pragma unroll
            for (int kb = 0; kb < 2; kb++)
#pragma unroll
                for (int nt = 0; nt < NT; nt++)
#pragma unroll
                    for (int mt = 0; mt < MT; mt++)
#pragma unroll
                        for (int v = 0; v < 4; v++)
                            acc[mt][nt][v] = fmaf(dsc[kb][nt], part[kb][mt][nt][v], acc[mt][nt][v]);
            __syncthreads();
        }
    }

    // D layout of a 16x16 tile: lane holds column lane & 15, rows 4 (lane >> 4) + v.
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int nt = 0; nt < NT; nt++)
#pragma unroll
            for (int v = 0; v < 4; v++) {
                const int m = m0 + wm * WM + mt * 16 + 4 * lk + v;
                const int n = n0 + wn * WN + nt * 16 + lr;
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
    // Large M: 128 x 64 tiles, register-pipelined (v == 2 forces it where the shape allows).
    if (aligned && v != 1 && N % kBigBN == 0 && K % 64 == 0 && (M >= 256 || v == 2) &&
        (int64_t)kBigBN * row_bytes < ((int64_t)1 << 31)) {
        const unsigned grid = (unsigned)(((M + kBigBM - 1) / kBigBM) * (N / kBigBN));
        const int nst = K / 64;
        const int cfg = tuning().gemm_big_config;
#define GOLLEK_BIG(P, WMW, WNW)                                                                \
    hipLaunchKernelGGL((gemm_q8_0_bf16_big_kernel<P, WMW, WNW>), dim3(grid),                \
                       dim3(64 * (WMW) * (WNW)), 0, stream, w, row_bytes, x, y, M, N, K)
        // Measured on MI355X (4096 x 4096, M = 256 .. 1024): the eight-wave
        // 2-deep pipeline (112 VGPRs, two workgroups per CU when the grid
        // has them) matches the deeper ones at M = 512 and wins at M = 1024.
        if (nst % 4 == 0 && cfg == 1) GOLLEK_BIG(4, 4, 2);
        else if (nst % 8 == 0 && cfg == 2) GOLLEK_BIG(8, 4, 2);
        else if (nst % 4 == 0 && cfg == 4) GOLLEK_BIG(4, 2, 2);
        else if (nst % 2 == 0) GOLLEK_BIG(2, 4, 2);
        else GOLLEK_BIG(1, 4, 2);
#undef GOLLEK_BIG
        return hipGetLastError();
    }
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
