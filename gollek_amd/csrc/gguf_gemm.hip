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
// Kernels.  M > 32: gemm_q8_0_bf16_ring_kernel (128 x 64 workgroup tiles
// fed by buffer->LDS loads, described below; when the tiles cover less than
// half the CUs, as for M <= 256 at N = 4096, each tile's K range is split
// over up to 8 workgroups whose partial tiles gemm_splitk_reduce_kernel sums
// in split order, so the result does not depend on timing;
// gemm_q8_0_bf16_big_kernel, the register-pipelined version of the same
// tiling, remains selectable).  M <= 32: gemm_q8_0_bf16_skinny_kernel
// (16-row column tiles, K split over the waves, one buffer->LDS ring per
// wave).  Other shapes and the sweep variants: gemm_q8_0_bf16_kernel, where
// a workgroup of 4 waves owns a BM x BN tile of Y; the waves split it WM x WN
// and, when WK > 1, also split each K stage (the partial tiles are summed
// through LDS at the end).  Each stage moves
// KB = 64 * WK columns of X (bf16) and W (Q8_0 block pairs, 68 aligned bytes,
// realigned and widened to bf16 once per workgroup) into double-buffered LDS;
// one barrier per stage.
#include <type_traits>

#include "gguf_blocks.hpp"
#include "gguf_dot4.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));

constexpr int kPad = 8;  // bf16 elements of row padding in LDS (bank spread)

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    // Exact: |q| <= 128 is representable in bf16 (one v_cvt_pk_bf16_f32).
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
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

// ---- large-M ring kernel --------------------------------------------------------
//
// Same 128 x 64 workgroup tile, eight waves of 32 x 32 and the same MFMA /
// scale arithmetic as gemm_q8_0_bf16_big_kernel, with the operands moved by
// buffer->LDS loads into a ring of six stage slots:
//   - X: the stage's 128 rows x 64 columns of bf16 land directly in the
//     XOR-swizzled layout of swz() (each lane loads the global chunk that
//     belongs at its LDS position);
//   - W: each row's 68-byte stage piece (a Q8_0 block pair) lands raw, its
//     dwords 0..15 as four 16-byte chunks and dword 16 in a separate array.
// The workgroup widens W to bf16 (and the block scales to fp32) two stages
// ahead into one of three converted-W buffers.  The work of stage s is spread
// so that the units overlap: right after the stage's one barrier each wave
// issues the MFMAs of stage s from fragments it read during stage s - 1,
// then the loads of stage s + 5, reads the fragments of stage s + 1, widens
// stage s + 2, and applies the block scales to the MFMA results of stage
// s - 1.  The loop is unrolled by the six slots so that every LDS address is
// a per-lane register plus an immediate.  The LDS reads of ring data and all
// LDS writes in the loop are inline asm: the compiler cannot tell which
// buffer->LDS load wrote which bytes and would otherwise wait for every load
// in flight.
//
// Default (LOADERS): two more waves issue every load of the ring and wait for
// them before each barrier, so the eight compute waves never stall at a load
// issue when the CU's queue of outstanding requests is full (measured on
// MI355X at M = 512: 36-37 us against 38-39 us with every wave loading).

namespace {

constexpr int kRgSlots = 6;
constexpr int kRgXBytes = kBigBM * kRowStride;                  // X stage (bf16, swizzled)
constexpr int kRgWQBytes = kBigBN * 64;                         // W dwords 0..15 per row
constexpr int kRgW16Bytes = kBigBN * 4;                         // W dword 16 per row
constexpr int kRgSlot = kRgXBytes + kRgWQBytes + kRgW16Bytes;   // 20736 bytes
constexpr int kRgWbBytes = kBigBN * kRowStride;                 // converted W (bf16, swizzled)
constexpr int kRgWbuf = kRgWbBytes + kBigBN * 8;                // + fp32 scales [row][2]
constexpr int kRgWbufs = 3;
constexpr int kRgDmaPerWave = 3;                                // 2 X + 1 W (or sink) per stage
constexpr int kRgLds = kRgSlots * kRgSlot + kRgWbufs * kRgWbuf + 256;
static_assert(kRgLds <= 160 * 1024, "LDS budget");
// Slots 0..2 and 3..5 are addressed from two base registers so that every
// offset fits the 16-bit immediate of the DS instructions.
static_assert(2 * kRgSlot + kRgSlot <= 65536, "slot group offsets");

// The stage's MFMA operands of one wave: A for blocks (kb) x rows (mt), B for
// blocks x columns (nt), and the fp32 scale pairs of its two 16-column groups.
struct RingFrags {
    u32x4 a00, a01, a10, a11;  // a[kb][mt]
    u32x4 b00, b01, b10, b11;  // b[kb][nt]
    uint2 d0, d1;              // {d[n][0], d[n][1]} for nt = 0, 1
};

// Issues the reads only: the registers are valid after ring_wait() names them.
template <int XO, int WO>
__device__ __forceinline__ void ring_read_frags(uint32_t xa0, uint32_t xa1, uint32_t wb0,
                                                uint32_t wb1, uint32_t dd, RingFrags &f) {
    asm volatile(
        "ds_read_b128 %0, %10 offset:%15\n\t"
        "ds_read_b128 %1, %10 offset:%16\n\t"
        "ds_read_b128 %2, %11 offset:%15\n\t"
        "ds_read_b128 %3, %11 offset:%16\n\t"
        "ds_read_b128 %4, %12 offset:%17\n\t"
        "ds_read_b128 %5, %12 offset:%18\n\t"
        "ds_read_b128 %6, %13 offset:%17\n\t"
        "ds_read_b128 %7, %13 offset:%18\n\t"
        "ds_read_b64 %8, %14 offset:%17\n\t"
        "ds_read_b64 %9, %14 offset:%19"
        : "=&v"(f.a00), "=&v"(f.a01), "=&v"(f.a10), "=&v"(f.a11), "=&v"(f.b00), "=&v"(f.b01),
          "=&v"(f.b10), "=&v"(f.b11), "=&v"(f.d0), "=&v"(f.d1)
        : "v"(xa0), "v"(xa1), "v"(wb0), "v"(wb1), "v"(dd), "n"(XO), "n"(XO + 2048), "n"(WO),
          "n"(WO + 2048), "n"(WO + 128)
        : "memory");
}

// Three raw dwords of a W piece (separate addresses: dword 16 lives apart)
// and the scale dword; issued only, valid after ring_wait().
template <int OFF>
__device__ __forceinline__ void ring_read_raw(uint32_t a0, uint32_t a1, uint32_t a2, uint32_t a3,
                                              uint32_t &d0, uint32_t &d1, uint32_t &d2,
                                              uint32_t &d3) {
    asm volatile(
        "ds_read_b32 %0, %4 offset:%8\n\t"
        "ds_read_b32 %1, %5 offset:%8\n\t"
        "ds_read_b32 %2, %6 offset:%8\n\t"
        "ds_read_b32 %3, %7 offset:%8"
        : "=&v"(d0), "=&v"(d1), "=&v"(d2), "=&v"(d3)
        : "v"(a0), "v"(a1), "v"(a2), "v"(a3), "n"(OFF)
        : "memory");
}

template <int OFF, typename T>
__device__ __forceinline__ void ring_read(uint32_t a, T &v) {
    if constexpr (sizeof(T) == 16)
        asm volatile("ds_read_b128 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
    else
        asm volatile("ds_read_b64 %0, %1 offset:%2" : "=v"(v) : "v"(a), "n"(OFF) : "memory");
}

// Waits for every LDS read in flight.  The registers the reads write pass
// through the statement, so no use of them can be scheduled before it.
__device__ __forceinline__ void ring_wait(RingFrags &f, uint32_t &d0, uint32_t &d1, uint32_t &d2,
                                          uint32_t &d3) {
    asm volatile("s_waitcnt lgkmcnt(0)"
                 : "+v"(f.a00), "+v"(f.a01), "+v"(f.a10), "+v"(f.a11), "+v"(f.b00), "+v"(f.b01),
                   "+v"(f.b10), "+v"(f.b11), "+v"(f.d0), "+v"(f.d1), "+v"(d0), "+v"(d1), "+v"(d2),
                   "+v"(d3)
                 :
                 : "memory");
}

template <int OFF>
__device__ __forceinline__ void ring_store4(uint32_t addr, u32x4 v) {
    asm volatile("ds_write_b128 %0, %1 offset:%2" : : "v"(addr), "v"(v), "n"(OFF) : "memory");
}

template <int OFF>
__device__ __forceinline__ void ring_store1(uint32_t addr, float v) {
    asm volatile("ds_write_b32 %0, %1 offset:%2" : : "v"(addr), "v"(v), "n"(OFF) : "memory");
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

}  // namespace

template <bool LOADERS>
__global__ __launch_bounds__(LOADERS ? 640 : 512) void gemm_q8_0_bf16_ring_kernel(const uint8_t *__restrict__ W,
                                                                  int64_t row_bytes,
                                                                  const uint16_t *__restrict__ X,
                                                                  float *__restrict__ Y, int M,
                                                                  int N, int K, int S,
                                                                  float *__restrict__ partials) {
    constexpr int NS = kRgSlots;
    __shared__ __attribute__((aligned(16))) uint8_t lds[kRgLds];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int wm = wave >> 1, wn = wave & 1;

    // Tile order: groups of up to four M tiles, N-major inside a group, so
    // that the workgroups an XCD runs at one time (the contiguous range
    // [j G/8, (j+1) G/8) when the grid divides by 8, workgroups being dealt
    // to XCDs round robin) share their X rows and W rows in that XCD's L2.
    // With S > 1 (split-K) the S workgroups of a tile are adjacent in this
    // order and split k takes stages [k nst, (k + 1) nst) of K, writing its
    // partial tile to partials[k] (summed in split order by a second kernel).
    const int m_tiles = (M + kBigBM - 1) / kBigBM;
    const int n_tiles = N / kBigBN;
    const int G = (int)gridDim.x;
    const int v = (G % 8 == 0) ? (int)(blockIdx.x % 8) * (G / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int t = v / S, split = v - t * S;
    const int group = t / (4 * n_tiles);
    const int first_m = 4 * group;
    const int gm = m_tiles - first_m < 4 ? m_tiles - first_m : 4;
    const int local = t - group * 4 * n_tiles;
    const int mt_idx = first_m + local % gm, nt_idx = local / gm;
    const int m0 = mt_idx * kBigBM, n0 = nt_idx * kBigBN;
    const int nst = K / 64 / S;
    const int s0 = split * nst;

    // X rows m0.. (zeros past M), W rows n0.. (N % 64 == 0 by dispatch), both
    // from the split's first column.  Loads of stages past the last one read
    // the following bytes of the same buffers (or zeros past their ends) into
    // slots that are never used.
    const __amdgpu_buffer_rsrc_t xs = wave_buffer(
        reinterpret_cast<const uint8_t *>(X) + (int64_t)m0 * K * 2 + (int64_t)s0 * 128,
        (uint32_t)((int64_t)(M - m0 < kBigBM ? M - m0 : kBigBM) * K * 2 - (int64_t)s0 * 128));
    const __amdgpu_buffer_rsrc_t ws = wave_buffer(W + (int64_t)n0 * row_bytes + (int64_t)s0 * 68,
                                                  (uint32_t)(kBigBN * row_bytes - (int64_t)s0 * 68));

    uint8_t *const sink = lds + NS * kRgSlot + kRgWbufs * kRgWbuf;
    const uint32_t base0 = (uint32_t)(uintptr_t)(lds_ptr)lds;
    const uint32_t base1 = base0 + 3u * kRgSlot;
    const uint32_t wbase = base0 + (uint32_t)(NS * kRgSlot);

    if constexpr (LOADERS) {
        if (wave >= 8) {
            // Loader waves (the eight compute waves issue no loads): wave 8
            // moves X chunks 0..9 and dword 16 of every W row, wave 9 X chunks
            // 10..15, the four W chunks and one sink load: 11 each per stage.
            const int lw = wave - 8;
            auto load_stage = [&](int st) {
                uint8_t *slot = lds + (st % NS) * kRgSlot;
                const uint32_t xk = (uint32_t)st * 128u, wk = (uint32_t)st * 68u;
                if (lw == 0) {
#pragma unroll
                    for (int c = 0; c < 10; c++) {
                        const int p = 64 * c + lane;
                        const int r = p >> 3, kc = (p & 7) ^ ((r >> 1) & 7);
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            xs, (lds_ptr)(slot + 1024 * c), 16,
                            (uint32_t)r * (uint32_t)(2 * K) + 16u * (uint32_t)kc + xk, 0, 0, 0);
                    }
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(ws, (lds_ptr)(slot + kRgXBytes + kRgWQBytes), 4,
                                                             (uint32_t)lane * (uint32_t)row_bytes + 64u + wk, 0,
                                                             0, 0);
                } else {
#pragma unroll
                    for (int c = 10; c < 16; c++) {
                        const int p = 64 * c + lane;
                        const int r = p >> 3, kc = (p & 7) ^ ((r >> 1) & 7);
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            xs, (lds_ptr)(slot + 1024 * c), 16,
                            (uint32_t)r * (uint32_t)(2 * K) + 16u * (uint32_t)kc + xk, 0, 0, 0);
                    }
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const int q = 64 * c + lane;
                        __builtin_amdgcn_raw_ptr_buffer_load_lds(
                            ws, (lds_ptr)(slot + kRgXBytes + 1024 * c), 16,
                            (uint32_t)(q >> 2) * (uint32_t)row_bytes + 16u * (uint32_t)(q & 3) + wk, 0, 0, 0);
                    }
                    __builtin_amdgcn_raw_ptr_buffer_load_lds(ws, (lds_ptr)sink, 4, kMaskedOffset, 0, 0, 0);
                }
            };
            for (int st = 0; st < NS - 1; st++) load_stage(st);
            // The compute waves' two prologue barriers: stages 0..2 landed,
            // then stages 0 and 1 widened.
            asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(11 * (NS - 3)) : "memory");
            asm volatile("s_barrier" ::: "memory");
            for (int st = 0; st < nst; st++) {
                // Stage st + 2 has landed; stage st - 1's slot is free.
                asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(11 * (NS - 4)) : "memory");
                load_stage(st + NS - 1);
            }
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            return;
        }
    }

    // Loads of a stage.  X: wave w moves LDS chunks 64 (2w + i) + lane of the
    // slot, i.e. row r = chunk / 8 at swizzled position chunk % 8, which holds
    // the row's 16-byte column chunk kc = position ^ ((r >> 1) & 7).  W: waves
    // 0..3 move 16-byte chunks (row = chunk / 4, part chunk % 4) of dwords
    // 0..15, wave 4 moves dword 16 of every row, waves 5..7 issue a masked
    // load into a sink so that every wave has the same count in flight.
    uint32_t xo[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const int p = 64 * (2 * wave + i) + lane;
        const int r = p >> 3, kc = (p & 7) ^ ((r >> 1) & 7);
        xo[i] = (uint32_t)r * (uint32_t)(2 * K) + 16u * (uint32_t)kc;
    }
    const int wp = 64 * wave + lane;
    const uint32_t wo = wave < 4 ? (uint32_t)(wp >> 2) * (uint32_t)row_bytes + 16u * (uint32_t)(wp & 3)
                                 : (uint32_t)lane * (uint32_t)row_bytes + 64u;
    auto issue_x = [&](int s, uint8_t *slot, int i) {
        __builtin_amdgcn_raw_ptr_buffer_load_lds(xs, (lds_ptr)(slot + 1024 * (2 * wave + i)), 16,
                                                 xo[i] + (uint32_t)s * 128u, 0, 0, 0);
    };
    auto issue_w = [&](int s, uint8_t *slot) {
        const uint32_t wk = (uint32_t)s * 68u;
        if (wave < 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ws, (lds_ptr)(slot + kRgXBytes + 1024 * wave), 16,
                                                     wo + wk, 0, 0, 0);
        else if (wave == 4)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ws, (lds_ptr)(slot + kRgXBytes + kRgWQBytes), 4,
                                                     wo + wk, 0, 0, 0);
        else
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ws, (lds_ptr)sink, 4, kMaskedOffset, 0, 0, 0);
    };
    auto issue = [&](int s, uint8_t *slot) {
        issue_x(s, slot, 0);
        issue_x(s, slot, 1);
        issue_w(s, slot);
    };

    // Widening role: row cn, block cb, quants 8 cu .. 8 cu + 7 of the block,
    // which start in raw dword i0 = 2 cu (block 0: at byte 2) or 9 + 2 cu
    // (block 1: aligned).  Dword 16 of a row lives in the separate array.
    // Waves 6 and 7 also widen the block-0 / block-1 scale of row `lane`.
    const int cn = tid >> 3, cb = (tid >> 2) & 1, cu = tid & 3;
    const int ci0 = cb ? 9 + 2 * cu : 2 * cu;
    const uint32_t csh = cb ? 0u : 2u;
    auto raw_at = [&](int i) {
        return (uint32_t)(i < 16 ? kRgXBytes + 64 * cn + 4 * i : kRgXBytes + kRgWQBytes + 4 * cn);
    };
    const uint32_t cr0 = raw_at(ci0), cr1 = raw_at(ci0 + 1), cr2 = raw_at(ci0 + 2);
    const uint32_t cr0_g[2] = {base0 + cr0, base1 + cr0}, cr1_g[2] = {base0 + cr1, base1 + cr1},
                   cr2_g[2] = {base0 + cr2, base1 + cr2};
    const uint32_t cw = wbase + swz(cn, 4 * cb + cu);
    const int sb = wave - 6;  // scale block of waves 6 and 7
    const uint32_t cs_g[2] = {base0 + (uint32_t)(kRgXBytes + 64 * lane + 32 * sb),
                              base1 + (uint32_t)(kRgXBytes + 64 * lane + 32 * sb)};
    const uint32_t cd = wbase + (uint32_t)(kRgWbBytes + 8 * lane + 4 * sb);
    // Waves below 6 read their first quant dword again instead of a scale.
    const uint32_t cs_g2[2] = {wave >= 6 ? cs_g[0] : cr0_g[0], wave >= 6 ? cs_g[1] : cr0_g[1]};
    uint32_t rw[4];
    auto widen_read = [&](auto SLOT) {
        constexpr int so = (decltype(SLOT)::value % 3) * kRgSlot;
        constexpr int g = decltype(SLOT)::value / 3;
        ring_read_raw<so>(cr0_g[g], cr1_g[g], cr2_g[g], cs_g2[g], rw[0], rw[1], rw[2], rw[3]);
    };
    auto widen_write = [&](auto WB) {
        constexpr int wbo = decltype(WB)::value * kRgWbuf;
        const uint32_t q0 = __builtin_amdgcn_alignbyte(rw[1], rw[0], csh);
        const uint32_t q1 = __builtin_amdgcn_alignbyte(rw[2], rw[1], csh);
        uint32_t o[4];
        i8x4_to_bf16(q0, o[0], o[1]);
        i8x4_to_bf16(q1, o[2], o[3]);
        ring_store4<wbo>(cw, u32x4{o[0], o[1], o[2], o[3]});
        if (wave >= 6) ring_store1<wbo>(cd, half_bits_to_float_fast(sb ? rw[3] >> 16 : rw[3] & 0xFFFFu));
    };

    // Fragment addresses (per lane; the slot / buffer offset is an immediate).
    const int lr = lane & 15, lk = lane >> 4;
    const uint32_t f_xa0 = swz(32 * wm + lr, lk), f_xa1 = swz(32 * wm + lr, 4 + lk);
    const uint32_t xa0_g[2] = {base0 + f_xa0, base1 + f_xa0}, xa1_g[2] = {base0 + f_xa1, base1 + f_xa1};
    const uint32_t wb0 = wbase + swz(32 * wn + lr, lk), wb1 = wbase + swz(32 * wn + lr, 4 + lk);
    const uint32_t wdd = wbase + (uint32_t)(kRgWbBytes + 8 * (32 * wn + lr));
    auto read_frags = [&](auto SLOT, auto WB, RingFrags &f) {
        constexpr int so = (decltype(SLOT)::value % 3) * kRgSlot;
        constexpr int g = decltype(SLOT)::value / 3;
        constexpr int wbo = decltype(WB)::value * kRgWbuf;
        ring_read_frags<so, wbo>(xa0_g[g], xa1_g[g], wb0, wb1, wdd, f);
    };

    f32x4 acc[2][2];
    f32x4 part[2][2][2][2];  // [set][kb][mt][nt]
    float dsc[2][2][2];      // [set][kb][nt]
#pragma unroll
    for (int a = 0; a < 2; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) {
            acc[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
            for (int c = 0; c < 2; c++) {
                part[1][c][a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
                dsc[1][c][a] = 0.0f;
            }
        }
    RingFrags F[2];

    auto mfma_one = [&](int set, const RingFrags &f, int q) {
        const int kb = q >> 2, mt = (q >> 1) & 1, nt = q & 1;
        const u32x4 a = kb ? (mt ? f.a11 : f.a10) : (mt ? f.a01 : f.a00);
        const u32x4 b = kb ? (nt ? f.b11 : f.b10) : (nt ? f.b01 : f.b00);
        part[set][kb][mt][nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(
            as_bf16x8(a), as_bf16x8(b), f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
    };
    auto scale_q = [&](int set, int q) {
        const int kb = q >> 2, nt = (q >> 1) & 1, mt = q & 1;
#pragma unroll
        for (int v = 0; v < 4; v++)
            acc[mt][nt][v] = fmaf(dsc[set][kb][nt], part[set][kb][mt][nt][v], acc[mt][nt][v]);
    };
    auto pin_acc = [&]() {
        asm volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[1][0]), "+v"(acc[1][1]));
    };
    auto scale = [&](int set) {
#pragma unroll
        for (int kb = 0; kb < 2; kb++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int mt = 0; mt < 2; mt++)
#pragma unroll
                    for (int v = 0; v < 4; v++)
                        acc[mt][nt][v] = fmaf(dsc[set][kb][nt], part[set][kb][mt][nt][v], acc[mt][nt][v]);
    };

    // Prologue: stages 0..4 in flight; stages 0 and 1 widened; fragments of 0 read.
    using I0 = std::integral_constant<int, 0>;
    using I1 = std::integral_constant<int, 1>;
    if constexpr (!LOADERS) {
        issue(0, lds);
        issue(1, lds + kRgSlot);
        issue(2, lds + 2 * kRgSlot);
        issue(3, lds + 3 * kRgSlot);
        issue(4, lds + 4 * kRgSlot);
    }
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(kRgDmaPerWave * (NS - 3)) : "memory");
    widen_read(I0{});
    ring_wait(F[1], rw[0], rw[1], rw[2], rw[3]);
    widen_write(I0{});
    widen_read(I1{});
    ring_wait(F[1], rw[0], rw[1], rw[2], rw[3]);
    widen_write(I1{});
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    read_frags(I0{}, I0{}, F[0]);
    ring_wait(F[0], rw[0], rw[1], rw[2], rw[3]);

    // Stage s = 6 c + j sits in slot j, its widened W in buffer s % 3 = j % 3.
    auto stage = [&](auto J, int s) {
        constexpr int j = decltype(J)::value;
        constexpr int cur = j & 1, nxt = cur ^ 1;
        // Stage s + 2 has landed for every wave; stage s + 1 is widened.
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier"
                     :
                     : "n"(kRgDmaPerWave * (NS - 4))
                     : "memory");
        // Eight groups, one MFMA of stage s each, with four scale FMAs of
        // stage s - 1 and the LDS reads of stages s + 2 (raw W) and s + 1
        // (fragments) or a load issue, so that the LDS, the matrix core, the
        // VALU and the load path each see a steady stream.
        constexpr int sn = (j + 1) % NS, gn = sn / 3, so_n = (sn % 3) * kRgSlot;
        constexpr int wo_n = ((j + 1) % 3) * kRgWbuf;
        constexpr int sd = (j + NS - 1) % NS;
        RingFrags &f = F[cur];
        RingFrags &fn = F[nxt];
        dsc[cur][0][0] = __uint_as_float(f.d0.x);
        dsc[cur][1][0] = __uint_as_float(f.d0.y);
        dsc[cur][0][1] = __uint_as_float(f.d1.x);
        dsc[cur][1][1] = __uint_as_float(f.d1.y);
        {
            widen_read(std::integral_constant<int, (j + 2) % NS>{});
            __builtin_amdgcn_sched_barrier(0);
            mfma_one(cur, f, 0);
            scale_q(nxt, 0);
            __builtin_amdgcn_sched_barrier(0);
            ring_read<so_n>(xa0_g[gn], fn.a00);
            ring_read<so_n + 2048>(xa0_g[gn], fn.a01);
            mfma_one(cur, f, 1);
            scale_q(nxt, 1);
            __builtin_amdgcn_sched_barrier(0);
            ring_read<so_n>(xa1_g[gn], fn.a10);
            ring_read<so_n + 2048>(xa1_g[gn], fn.a11);
            mfma_one(cur, f, 2);
            scale_q(nxt, 2);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (!LOADERS) issue_x(s + NS - 1, lds + sd * kRgSlot, 0);
            else asm volatile("" ::: "memory");
            ring_read<wo_n>(wb0, fn.b00);
            ring_read<wo_n + 2048>(wb0, fn.b01);
            mfma_one(cur, f, 3);
            scale_q(nxt, 3);
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (!LOADERS) issue_x(s + NS - 1, lds + sd * kRgSlot, 1);
            else asm volatile("" ::: "memory");
            ring_read<wo_n>(wb1, fn.b10);
            ring_read<wo_n + 2048>(wb1, fn.b11);
            mfma_one(cur, f, 4);
            scale_q(nxt, 4);
            pin_acc();
            __builtin_amdgcn_sched_barrier(0);
            if constexpr (!LOADERS) issue_w(s + NS - 1, lds + sd * kRgSlot);
            else asm volatile("" ::: "memory");
            __builtin_amdgcn_sched_barrier(0);
            ring_read<wo_n>(wdd, fn.d0);
            ring_read<wo_n + 128>(wdd, fn.d1);
            mfma_one(cur, f, 5);
            scale_q(nxt, 5);
            __builtin_amdgcn_sched_barrier(0);
            mfma_one(cur, f, 6);
            scale_q(nxt, 6);
            __builtin_amdgcn_sched_barrier(0);
            mfma_one(cur, f, 7);
            scale_q(nxt, 7);
            pin_acc();
            __builtin_amdgcn_sched_barrier(0);
            ring_wait(F[nxt], rw[0], rw[1], rw[2], rw[3]);
            widen_write(std::integral_constant<int, (j + 2) % 3>{});
        }
        if (s + 1 == nst) scale(cur);
    };
    for (int s = 0; s < nst; s += NS) {
        stage(std::integral_constant<int, 0>{}, s);
        if (s + 1 >= nst) break;
        stage(std::integral_constant<int, 1>{}, s + 1);
        if (s + 2 >= nst) break;
        stage(std::integral_constant<int, 2>{}, s + 2);
        if (s + 3 >= nst) break;
        stage(std::integral_constant<int, 3>{}, s + 3);
        if (s + 4 >= nst) break;
        stage(std::integral_constant<int, 4>{}, s + 4);
        if (s + 5 >= nst) break;
        stage(std::integral_constant<int, 5>{}, s + 5);
    }
    // Drain the loads issued past the last stage before the workgroup ends.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");

    // D layout of a 16x16 tile: lane holds column lane & 15, rows 4 (lane >> 4) + v.
    float *const out = partials != nullptr ? partials + (int64_t)split * M * N : Y;
#pragma unroll
    for (int mt = 0; mt < 2; mt++)
#pragma unroll
        for (int nt = 0; nt < 2; nt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 32 * wm + 16 * mt + 4 * lk + r;
                const int n = n0 + 32 * wn + 16 * nt + lr;
                if (m < M) out[(int64_t)m * N + n] = acc[mt][nt][r];
            }
}

// y = part[0] + part[1] + ... + part[S - 1], in that order (4 floats a
// thread, S <= 8): every partial is loaded before the first add, so the
// reduction costs one memory round trip.
__global__ __launch_bounds__(256) void gemm_splitk_reduce_kernel(const float *__restrict__ part, int S,
                                                                 int64_t mn, float *__restrict__ y) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= mn) return;
    // only the S partials are read (S is uniform); the sum runs in split order
    float4 b[8];
#pragma unroll
    for (int k = 0; k < 8; k++)
        if (k < S) b[k] = *reinterpret_cast<const float4 *>(part + (int64_t)k * mn + i);
    float4 a = b[0];
#pragma unroll
    for (int k = 1; k < 8; k++) {
        if (k < S) {
            a.x += b[k].x;
            a.y += b[k].y;
            a.z += b[k].z;
            a.w += b[k].w;
        }
    }
    *reinterpret_cast<float4 *>(y + i) = a;
}

// ---- small-M ring kernel --------------------------------------------------------
//
// M <= 16 TT tokens.  A workgroup of four waves owns 16 W rows and every
// token.  Wave w contracts the Q8_0 block pairs p = w, w + 4, w + 8, ... of
// K (64 columns each) and has a ring of NS slots of its own, so the waves
// never wait for each other until the end: per pair it loads, by
// buffer->LDS, the tokens' 64 bf16 columns (16-byte chunks XOR-swizzled by
// token pair, so the fragment reads are free of bank conflicts) and the 16
// rows' 68-byte raw pieces (dwords 0..15 as 16-byte chunks, dword 16 apart).
// X is the MFMA A operand (rows = tokens) and W the B operand, widened from
// the raw quants in registers: each lane's output column is one W row, so a
// block scale is one value per lane.  The four waves' partial tiles are
// summed through LDS in wave order at the end.

namespace {

constexpr int kSkRows = 16;

template <int TT>
struct SkGeom {
    static constexpr int kXBytes = 16 * TT * 128;   // tokens x 64 bf16
    static constexpr int kWQ = kXBytes;             // 16 rows x dwords 0..15
    static constexpr int kW16 = kWQ + 1024;         // dword 16 of each row (64 lanes x 4 B)
    static constexpr int kSlot = kW16 + 256;
    static constexpr int kXDma = TT * 2;
    static constexpr int kDma = kXDma + 2;          // + W chunks + W dword 16
};

template <int TT, int NS>
constexpr int skinny_lds_bytes() {
    return 4 * NS * SkGeom<TT>::kSlot + 3 * TT * 1024;
}

// 16- and 4-byte-per-lane buffer->LDS loads (__device__ functions: called
// directly from a kernel template's body, the builtin makes hipcc's host pass
// drop the kernel's launch stub).
__device__ __forceinline__ void dma_lds16(__amdgpu_buffer_rsrc_t rs, uint8_t *dst, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)dst, 16, off, 0, 0, 0);
}
__device__ __forceinline__ void dma_lds4(__amdgpu_buffer_rsrc_t rs, uint8_t *dst, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)dst, 4, off, 0, 0, 0);
}

// s_waitcnt vmcnt(N) (a separate template: an asm immediate that depends on
// a kernel template's parameters also drops the stub).
template <int N>
__device__ __forceinline__ void wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// One pair's LDS reads of a wave: raw dwords 2kq, 2kq + 1, 2kq + 2, 9 + 2kq
// (from wr0), 10 + 2kq (w10a: dword 16 lives apart), scale dwords 0 and 8
// (from wrs), and the X fragments of both blocks and TT token tiles.
template <int TT>
__device__ __forceinline__ void skinny_read(uint32_t wr0, uint32_t w10a, uint32_t wrs, uint32_t xa0,
                                            uint32_t xa1, uint2 &w01, uint2 &w29, uint32_t &w10,
                                            uint2 &sc, u32x4 (&xf)[2][TT]) {
    if constexpr (TT == 1) {
        asm volatile(
            "ds_read2_b32 %0, %6 offset0:0 offset1:1\n\t"
            "ds_read2_b32 %1, %6 offset0:2 offset1:9\n\t"
            "ds_read_b32 %2, %7\n\t"
            "ds_read2_b32 %3, %8 offset0:0 offset1:8\n\t"
            "ds_read_b128 %4, %9\n\t"
            "ds_read_b128 %5, %10\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w01), "=&v"(w29), "=&v"(w10), "=&v"(sc), "=&v"(xf[0][0]), "=&v"(xf[1][0])
            : "v"(wr0), "v"(w10a), "v"(wrs), "v"(xa0), "v"(xa1)
            : "memory");
    } else {
        asm volatile(
            "ds_read2_b32 %0, %8 offset0:0 offset1:1\n\t"
            "ds_read2_b32 %1, %8 offset0:2 offset1:9\n\t"
            "ds_read_b32 %2, %9\n\t"
            "ds_read2_b32 %3, %10 offset0:0 offset1:8\n\t"
            "ds_read_b128 %4, %11\n\t"
            "ds_read_b128 %5, %11 offset:2048\n\t"
            "ds_read_b128 %6, %12\n\t"
            "ds_read_b128 %7, %12 offset:2048\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(w01), "=&v"(w29), "=&v"(w10), "=&v"(sc), "=&v"(xf[0][0]), "=&v"(xf[0][TT - 1]),
              "=&v"(xf[1][0]), "=&v"(xf[1][TT - 1])
            : "v"(wr0), "v"(w10a), "v"(wrs), "v"(xa0), "v"(xa1)
            : "memory");
    }
}

}  // namespace

template <int TT, int NS>
__global__ __launch_bounds__(256) void gemm_q8_0_bf16_skinny_kernel(const uint8_t *__restrict__ W,
                                                                    int64_t row_bytes,
                                                                    const uint16_t *__restrict__ X,
                                                                    float *__restrict__ Y, int M,
                                                                    int N, int K) {
    using G = SkGeom<TT>;
    __shared__ __attribute__((aligned(16))) uint8_t lds[skinny_lds_bytes<TT, NS>()];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = (int)blockIdx.x * kSkRows;
    const int npairs = K / 256;  // pairs per wave
    const int mrows = M < 16 * TT ? M : 16 * TT;

    // Tokens 0 .. mrows - 1 (zeros past M), W rows n0 .. n0 + 15.  Loads of
    // pairs past the last one read the following bytes of the same buffers
    // (or zeros past their ends) into slots that are never used.
    const __amdgpu_buffer_rsrc_t xs =
        wave_buffer(reinterpret_cast<const uint8_t *>(X), (uint32_t)((int64_t)mrows * K * 2));
    const __amdgpu_buffer_rsrc_t ws =
        wave_buffer(W + (int64_t)n0 * row_bytes, (uint32_t)(kSkRows * row_bytes));
    uint8_t *const ring = lds + wave * NS * G::kSlot;
    float *const red = reinterpret_cast<float *>(lds + 4 * NS * G::kSlot);

    // Load offsets of pair 0 (pair p adds 128 p to X, 68 p to W).  X: LDS
    // chunk q = 64 i + lane is token t = q / 8 at swizzled position q % 8,
    // which holds column chunk position ^ ((t >> 1) & 7).  W: chunk lane is
    // row lane / 4, part lane % 4; dword 16 of row lane (lanes < 16).
    uint32_t xo[2 * TT];
#pragma unroll
    for (int i = 0; i < 2 * TT; i++) {
        const int q = 64 * i + lane;
        const int t = q >> 3, c = (q & 7) ^ ((t >> 1) & 7);
        xo[i] = (uint32_t)t * (uint32_t)(2 * K) + 16u * (uint32_t)c;
    }
    const uint32_t wo = (uint32_t)(lane >> 2) * (uint32_t)row_bytes + 16u * (uint32_t)(lane & 3);
    const uint32_t w16o = lane < 16 ? (uint32_t)lane * (uint32_t)row_bytes + 64u : kMaskedOffset;
    auto issue = [&](int j, uint8_t *slot) {
        const uint32_t p = (uint32_t)(wave + 4 * j);
#pragma unroll
        for (int i = 0; i < 2 * TT; i++) dma_lds16(xs, slot + 1024 * i, xo[i] + 128u * p);
        dma_lds16(ws, slot + G::kWQ, wo + 68u * p);
        dma_lds4(ws, slot + G::kW16, lane < 16 ? w16o + 68u * p : kMaskedOffset);
    };

    // Fragment addresses relative to a slot.  A (X): token m = lane & 15 (+16
    // per token tile), chunk 4 kb + kq at its swizzled position.  B (W): row
    // n = lane & 15, quants 8 kq .. 8 kq + 7 of block kb (raw dwords 2kq ..
    // 2kq + 2 with block 0 starting at byte 2; 9 + 2kq, 10 + 2kq), scales in
    // dword 0 (low half) and dword 8 (high half).
    const int lr = lane & 15, kq = lane >> 4;
    const uint32_t xa0 = (uint32_t)(128 * lr + 16 * ((kq) ^ ((lr >> 1) & 7)));
    const uint32_t xa1 = (uint32_t)(128 * lr + 16 * ((4 + kq) ^ ((lr >> 1) & 7)));
    const uint32_t wr0 = (uint32_t)(G::kWQ + 64 * lr + 8 * kq);
    const uint32_t w10 = kq < 3 ? wr0 + 40u : (uint32_t)(G::kW16 + 4 * lr);
    const uint32_t wrs = (uint32_t)(G::kWQ + 64 * lr);
    const uint32_t ring_base = (uint32_t)(uintptr_t)(lds_ptr)ring;

    f32x4 acc[TT];
#pragma unroll
    for (int t = 0; t < TT; t++) acc[t] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};

#pragma unroll
    for (int j = 0; j < NS - 1; j++) issue(j, ring + j * G::kSlot);

    int sl = 0;
    for (int j = 0; j < npairs; j++) {
        wait_vm<G::kDma * (NS - 2)>();  // pair j has landed
        issue(j + NS - 1, ring + (sl == 0 ? NS - 1 : sl - 1) * G::kSlot);
        const uint32_t sb = ring_base + (uint32_t)(sl * G::kSlot);
        uint2 w01, w29, sc;
        uint32_t w10v;
        u32x4 xf[2][TT];
        skinny_read<TT>(sb + wr0, sb + w10, sb + wrs, sb + xa0, sb + xa1, w01, w29, w10v, sc, xf);
        uint32_t b0[4], b1[4];
        i8x4_to_bf16(__builtin_amdgcn_alignbyte(w01.y, w01.x, 2), b0[0], b0[1]);
        i8x4_to_bf16(__builtin_amdgcn_alignbyte(w29.x, w01.y, 2), b0[2], b0[3]);
        i8x4_to_bf16(w29.y, b1[0], b1[1]);
        i8x4_to_bf16(w10v, b1[2], b1[3]);
        const float d0 = half_bits_to_float_fast(sc.x & 0xFFFFu);
        const float d1 = half_bits_to_float_fast(sc.y >> 16);
        const bf16x8 B0 = as_bf16x8(u32x4{b0[0], b0[1], b0[2], b0[3]});
        const bf16x8 B1 = as_bf16x8(u32x4{b1[0], b1[1], b1[2], b1[3]});
#pragma unroll
        for (int t = 0; t < TT; t++) {
            const f32x4 p0 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xf[0][t]), B0,
                                                                     f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
            const f32x4 p1 = __builtin_amdgcn_mfma_f32_16x16x32_bf16(as_bf16x8(xf[1][t]), B1,
                                                                     f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
#pragma unroll
            for (int v = 0; v < 4; v++) acc[t][v] = fmaf(d1, p1[v], fmaf(d0, p0[v], acc[t][v]));
        }
        sl = sl + 1 == NS ? 0 : sl + 1;
    }
    // Drain the loads issued past the last pair, then sum the four waves'
    // partial tiles in wave order.  D layout of a 16x16 tile: lane holds
    // column lane & 15 (a W row), rows (tokens) 4 (lane >> 4) + v.
    wait_vm<0>();
    if (wave > 0) {
#pragma unroll
        for (int t = 0; t < TT; t++)
            *reinterpret_cast<f32x4 *>(red + (((wave - 1) * TT + t) * 64 + lane) * 4) = acc[t];
    }
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int t = 0; t < TT; t++) {
        f32x4 v = acc[t];
#pragma unroll
        for (int w = 0; w < 3; w++) v += *reinterpret_cast<const f32x4 *>(red + ((w * TT + t) * 64 + lane) * 4);
#pragma unroll
        for (int r = 0; r < 4; r++) {
            const int m = 16 * t + 4 * kq + r;
            if (m < M) Y[(int64_t)m * N + n0 + lr] = v[r];
        }
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

namespace {

// Splits of K for the large-M ring kernel: enough that the workgroups cover
// the CUs (up to 8), dividing the K stages evenly.
int ring_splits(int M, int N, int K) {
    const int tiles = (M + kBigBM - 1) / kBigBM * (N / kBigBN);
    const int nst = K / 64;
    int S = 1;
    while (S < 8 && tiles * 2 * S <= device_cus() && nst % (2 * S) == 0) S *= 2;
    return S;
}

bool ring_applies(int M, int N, int K, int64_t row_bytes) {
    return N % kBigBN == 0 && K % 64 == 0 && (int64_t)kBigBN * row_bytes < ((int64_t)1 << 31) &&
           (int64_t)kBigBM * K * 2 < ((int64_t)1 << 31);
}

}  // namespace

size_t gemm_workspace_bytes(int M, int N, int K) {
    if (M <= 32 || N % kBigBN != 0 || K % 64 != 0) return 0;
    const int S = ring_splits(M, N, K);
    return S > 1 ? (size_t)S * M * N * sizeof(float) : 0;
}

// The need of m peaks at multiples of the 128-row tile and is zero once the
// tiles cover half the CUs; S tiles <= cu_count (ring_splits) bounds it by
// cu_count tiles of 128 x 64 floats (8 MiB on 256 CUs, at m = 128).
size_t gemm_workspace_max_bytes(int N, int K) {
    size_t most = 0;
    for (int mt = 1; gemm_workspace_bytes(128 * mt, N, K) > 0; mt++) {
        const size_t b = gemm_workspace_bytes(128 * mt, N, K);
        if (b > most) most = b;
    }
    return most;
}

hipError_t launch_gemm_q8_0_bf16(const uint8_t *w, int64_t row_bytes, const uint16_t *x, float *y,
                                 int M, int N, int K, hipStream_t stream, float *workspace,
                                 size_t workspace_bytes) {
    if (M <= 0) return hipSuccess;
    const bool aligned = (reinterpret_cast<uintptr_t>(w) & 3u) == 0 && (row_bytes & 3) == 0 &&
                         (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    const int v = tuning().gemm_variant;
    // M > 32: 128 x 64 tiles (v == 2 forces them where the shape allows, v == 3
    // keeps the register-pipelined LDS tiles below M = 256), split over K
    // when the tiles alone leave CUs idle and a workspace is given.
    if (aligned && v != 1 && ring_applies(M, N, K, row_bytes) && (M >= 256 || v == 2 || (M > 32 && v != 3))) {
        const unsigned tiles = (unsigned)(((M + kBigBM - 1) / kBigBM) * (N / kBigBN));
        const unsigned grid = tiles;
        const int nst = K / 64;
        const int cfg = tuning().gemm_big_config;
        int S = ring_splits(M, N, K);
        // The reduction moves 16-byte vectors of y and the workspace.
        if (S > 1 && (workspace == nullptr || workspace_bytes < (size_t)S * M * N * sizeof(float) ||
                      ((reinterpret_cast<uintptr_t>(workspace) | reinterpret_cast<uintptr_t>(y)) & 15u) != 0))
            S = 1;
#define GOLLEK_BIG(P, WMW, WNW)                                                                \
    hipLaunchKernelGGL((gemm_q8_0_bf16_big_kernel<P, WMW, WNW>), dim3(grid),                \
                       dim3(64 * (WMW) * (WNW)), 0, stream, w, row_bytes, x, y, M, N, K)
        // Configs 1..4 select the register-pipelined kernel (sweeps); the
        // default is the buffer->LDS ring.
        if (nst % 4 == 0 && cfg == 1) GOLLEK_BIG(4, 4, 2);
        else if (nst % 8 == 0 && cfg == 2) GOLLEK_BIG(8, 4, 2);
        else if (nst % 2 == 0 && cfg == 3) GOLLEK_BIG(2, 4, 2);
        else if (nst % 4 == 0 && cfg == 4) GOLLEK_BIG(4, 2, 2);
        else {
            if (cfg == 5)
                hipLaunchKernelGGL(gemm_q8_0_bf16_ring_kernel<false>, dim3(tiles * S), dim3(512), 0, stream, w,
                                   row_bytes, x, y, M, N, K, S, S > 1 ? workspace : nullptr);
            else
                hipLaunchKernelGGL(gemm_q8_0_bf16_ring_kernel<true>, dim3(tiles * S), dim3(640), 0, stream, w,
                                   row_bytes, x, y, M, N, K, S, S > 1 ? workspace : nullptr);
            if (S > 1) {
                const int64_t mn = (int64_t)M * N;
                hipLaunchKernelGGL(gemm_splitk_reduce_kernel, dim3((unsigned)((mn / 4 + 255) / 256)),
                                   dim3(256), 0, stream, workspace, S, mn, y);
            }
        }
#undef GOLLEK_BIG
        return hipGetLastError();
    }
    // Small M: the buffer->LDS ring over 16-row column tiles (v == 3 keeps
    // the register-pipelined tiles below, for sweeps).
    if (aligned && v != 1 && v != 3 && M <= 32 && N % 16 == 0 && K % 256 == 0 &&
        (int64_t)16 * row_bytes < ((int64_t)1 << 31) && (int64_t)M * K * 2 < ((int64_t)1 << 31)) {
        const int cfg = tuning().gemm_big_config;
#define GOLLEK_SKINNY(TT, NS)                                                                      \
    hipLaunchKernelGGL((gemm_q8_0_bf16_skinny_kernel<TT, NS>), dim3(N / 16), dim3(256), 0, stream, w, \
                       row_bytes, x, y, M, N, K)
        // Measured on MI355X (4096 x 4096): four slots per wave beat deeper
        // rings (which only queue more requests at the HBM).
        if (M <= 16 && cfg == 18) GOLLEK_SKINNY(1, 8);
        else if (M <= 16) GOLLEK_SKINNY(1, 4);
        else GOLLEK_SKINNY(2, 4);
#undef GOLLEK_SKINNY
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
