// gguf_gemm.hip -- small-M GEMM (prefill / batched decode) dispatch, the
// Q8_0 kernels for M <= 32 and the fallbacks for other shapes, on gfx950.
//
// Y[M, N] = X[M, K] . W[N, K]^T with X bf16 and W a GGUF matrix (the Linear
// convention of runner/safetensor/gollek-safetensor-core/src/main/java/
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
// Kernels.  Q8_0 with M <= 32: gemm_q8_0_bf16_skinny_kernel (16-row column
// tiles, K split over the waves, one buffer->LDS ring per wave).  Q8_0, Q4_0
// and Q4_K with K a multiple of 256 otherwise: the 128 x 128 tile kernel of
// gguf_gemm_tile.hip.  Other shapes: gemm_q8_0_bf16_kernel, where a
// workgroup of 4 waves owns a BM x BN tile of Y; the waves split it WM x WN
// and, when WK > 1, also split each K stage (the partial tiles are summed
// through LDS at the end).  Each stage moves KB = 64 * WK columns of X (bf16)
// and W (Q8_0 block pairs, 68 aligned bytes, realigned and widened to bf16
// once per workgroup) into double-buffered LDS; one barrier per stage.  Any
// remaining shape or alignment: one thread per output (gemm_q8_0_generic_kernel,
// gemm_generic_kernel).
#include <type_traits>

#include "gguf_block_dot.hpp"
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

namespace {

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

}  // namespace

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

// Any shape, Q4_0 or Q4_K: one thread per output, fp32, the reference's block
// structure (Q4_0: d * sum((q - 8) x); Q4_K per sub-block: fl(d sc) sum(q x) -
// fl(dmin m) sum(x), the min term skipped for a zero min code).
template <int T>
__global__ __launch_bounds__(256) void gemm_generic_kernel(const uint8_t *__restrict__ W, int64_t row_bytes,
                                                           const uint16_t *__restrict__ X, float *__restrict__ Y,
                                                           int M, int N, int K) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)M * N) return;
    const int m = (int)(t / N), n = (int)(t - (int64_t)m * N);
    const uint8_t *row = W + (int64_t)n * row_bytes;
    const uint16_t *xr = X + (int64_t)m * K;
    auto xv = [&](int k) { return __uint_as_float((uint32_t)xr[k] << 16); };
    float acc = 0.0f;
    if constexpr (T == kQ4_0) {
        for (int b = 0; b < K / 32; b++) {
            const uint8_t *blk = row + (int64_t)b * kQ4BlockBytes;
            const float d = half_bits_to_float_fast((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
            float s = 0.0f;
            for (int i = 0; i < 16; i++) {
                const int q = blk[2 + i];
                s = fmaf((float)((q & 15) - 8), xv(32 * b + i), s);
                s = fmaf((float)((q >> 4) - 8), xv(32 * b + 16 + i), s);
            }
            acc = fmaf(d, s, acc);
        }
    } else {
        for (int sb = 0; sb < K / kQK; sb++) {
            const uint8_t *blk = row + (int64_t)sb * kQKBlockBytes;
            const float d = half_bits_to_float_fast((uint32_t)blk[0] | ((uint32_t)blk[1] << 8));
            const float dmin = half_bits_to_float_fast((uint32_t)blk[2] | ((uint32_t)blk[3] << 8));
            for (int j = 0; j < 8; j++) {
                int sc, mc;
                q4k_code(blk + 4, j, &sc, &mc);
                const uint8_t *q = blk + 16 + 32 * (j >> 1);
                const int sh = 4 * (j & 1);
                float s = 0.0f, sx = 0.0f;
                for (int i = 0; i < 32; i++) {
                    const float x = xv(kQK * sb + 32 * j + i);
                    s = fmaf((float)((q[i] >> sh) & 15), x, s);
                    sx += x;
                }
                acc = fmaf(d * (float)sc, s, acc);
                if (mc != 0) acc = fmaf(-(dmin * (float)mc), sx, acc);
            }
        }
    }
    Y[(int64_t)m * N + n] = acc;
}

// Q5_K / Q6_K: 16 x 16 outputs per workgroup, one per thread.  Per
// superblock the 16 X rows' 256 values (as fp32) and the 16 W rows'
// superblocks are staged in LDS, then each output adds its block's
// generic_block_dot (the dequantizers' block formulas folded into a dot;
// gguf_block_dot.hpp) in superblock order.
template <int T>
__global__ __launch_bounds__(256) void gemm_kquant_generic_kernel(const uint8_t *__restrict__ W,
                                                                  int64_t row_bytes,
                                                                  const uint16_t *__restrict__ X,
                                                                  float *__restrict__ Y, int M, int N, int K) {
    constexpr int PB = T == kQ6_K ? 210 : kQ5KBlockBytes;
    __shared__ float xs[16][kQK];
    __shared__ uint8_t ws[16][PB];
    const int n0 = (int)blockIdx.x * 16, m0 = (int)blockIdx.y * 16;
    const int tid = (int)threadIdx.x, n = tid & 15, m = tid >> 4;
    float acc = 0.0f;
    for (int sb = 0; sb < K / kQK; sb++) {
        __syncthreads();
        for (int i = tid; i < 16 * kQK; i += 256) {
            const int r = i / kQK, c = i - r * kQK;
            xs[r][c] = m0 + r < M ? __uint_as_float((uint32_t)X[(int64_t)(m0 + r) * K + kQK * sb + c] << 16) : 0.0f;
        }
        for (int i = tid; i < 16 * PB; i += 256) {
            const int r = i / PB, c = i - r * PB;
            ws[r][c] = n0 + r < N ? W[(int64_t)(n0 + r) * row_bytes + (int64_t)PB * sb + c] : (uint8_t)0;
        }
        __syncthreads();
        acc += generic_block_dot(T, ws[n], xs[m]);
    }
    if (m0 + m < M && n0 + n < N) Y[(int64_t)(m0 + m) * N + n0 + n] = acc;
}

// Q6_K on the matrix cores in fp32: a workgroup owns 16 NT W rows and 16 MT
// rows of X and walks K a superblock (256 columns) at a time.  Per
// stage the W rows' 210-byte superblocks and the X rows' bf16 go to LDS
// (both loaded into registers while the previous stage is contracted), the
// W values are dequantized there in fp32 -- d sc (q - 32) is exact in fp32
// (an 11-bit d times an 8-bit scale times a 6-bit code), so these are the
// dequantizer's values (RT/GgufKBlockDequantizer.java Q6_K: element e's
// code is a ql nibble and two qh bits, its scale the int8 of its 16) -- and
// contracted with v_mfma_f32_16x16x4_f32.  NT = 4 (tiles of 64 X rows): wave
// w owns W rows 16 w .. 16 w + 15 over all of the stage's columns, so X is
// staged once for 64 W rows.  NT = 1 (up to 32 X rows): wave w takes a
// quarter of the stage's columns and the four waves' sums meet in LDS in
// wave order.  X rows must be 4-byte aligned and W 2-byte aligned
// (launch_gemm_bf16 checks): W rows are read 2 bytes at a time (superblocks
// start on even bytes).
template <int MT, int NT>
__global__ __launch_bounds__(256) void gemm_q6k_f32_kernel(const uint8_t *__restrict__ W, int64_t row_bytes,
                                                           const uint16_t *__restrict__ X, float *__restrict__ Y,
                                                           int M, int N, int K) {
#pragma clang fp contract(off)
    static_assert(NT == 1 || NT == 4, "one N tile split over the waves, or one per wave");
    constexpr int BM = 16 * MT, BN = 16 * NT;
    constexpr int SBS = 1;                       // superblocks per stage
    constexpr int KS = kQK * SBS;                // columns per stage
    constexpr int kPitch = KS + 4;                // floats per staged row (bank spread)
    constexpr int kRowHalves = 105 * SBS;         // a W row's stage bytes as uint16
    constexpr int kRawHalves = BN * kRowHalves;
    constexpr int kRawPer = (kRawHalves + 255) / 256;
    constexpr int kXDw = BM * KS / 2;             // the X rows' stage as dwords
    constexpr int kXPer = kXDw / 256;
    constexpr int kGroups = BN * KS / 16;         // scale groups of the stage
    static_assert(kXDw % 256 == 0 && kGroups % 256 == 0, "whole rounds of the workgroup");
    __shared__ float xs[BM][kPitch];
    __shared__ float ws[BN][kPitch];
    __shared__ uint16_t raw[kRawHalves];
    __shared__ f32x4 red[NT == 1 ? 4 : 1][MT][64];
    const int tid = (int)threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n0 = (int)blockIdx.x * BN, m0 = (int)blockIdx.y * BM;
    const int nst = K / KS;
    uint16_t wr[kRawPer];
    uint32_t xr[kXPer];
    auto load = [&](int st) {
#pragma unroll
        for (int i = 0; i < kRawPer; i++) {
            const int h = tid + 256 * i, r = h / kRowHalves, c = h - r * kRowHalves;
            wr[i] = h < kRawHalves && n0 + r < N
                        ? *reinterpret_cast<const uint16_t *>(W + (int64_t)(n0 + r) * row_bytes +
                                                              (int64_t)(210 * SBS) * st + 2 * c)
                        : (uint16_t)0;
        }
#pragma unroll
        for (int i = 0; i < kXPer; i++) {
            const int q = tid + 256 * i, r = q / (KS / 2), c = q - r * (KS / 2);
            xr[i] = m0 + r < M ? *reinterpret_cast<const uint32_t *>(X + (int64_t)(m0 + r) * K + (int64_t)KS * st + 2 * c)
                               : 0u;
        }
    };
    f32x4 acc[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) acc[mt] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    load(0);
    for (int st = 0; st < nst; st++) {
        __syncthreads();  // the previous stage's LDS reads are done
#pragma unroll
        for (int i = 0; i < kRawPer; i++)
            if (tid + 256 * i < kRawHalves) raw[tid + 256 * i] = wr[i];
#pragma unroll
        for (int i = 0; i < kXPer; i++) {
            const int q = tid + 256 * i, r = q / (KS / 2), c = q - r * (KS / 2);
            xs[r][2 * c] = __uint_as_float(xr[i] << 16);
            xs[r][2 * c + 1] = __uint_as_float(xr[i] & 0xFFFF0000u);
        }
        __syncthreads();
        if (st + 1 < nst) load(st + 1);
        // group u: W row u / (16 SBS), superblock (u / 16) % SBS, its 16
        // elements of scale group u % 16
#pragma unroll
        for (int u = tid; u < kGroups; u += 256) {
            const int r = u / (16 * SBS), sb = (u / 16) % SBS, gi = u & 15;
            const uint8_t *b = reinterpret_cast<const uint8_t *>(raw) + 2 * kRowHalves * r + 210 * sb;
            const float d = half_bits_to_float((uint32_t)b[208] | ((uint32_t)b[209] << 8));
            const float dsc = d * (float)(int)(int8_t)b[192 + gi];
            const int e0 = 16 * gi, h = e0 >> 7, j = (e0 >> 5) & 3, l0 = e0 & 31;
#pragma unroll
            for (int i = 0; i < 16; i++) {
                const int l = l0 + i;
                const int q = ((b[64 * h + 32 * (j & 1) + l] >> (4 * (j >> 1))) & 0x0F) |
                              (((b[128 + 32 * h + l] >> (2 * j)) & 3) << 4);
                ws[r][kQK * sb + e0 + i] = dsc * (float)(q - 32);
            }
        }
        __syncthreads();
        const int col = lane & 15;
        // NT = 4: W rows of this wave's tile, every column; NT = 1: a quarter of the columns
        const int wrow = NT == 4 ? 16 * wave + col : col;
        const int kb = (NT == 4 ? 0 : (KS / 4) * wave) + (lane >> 4);
        constexpr int kSteps = NT == 4 ? KS / 4 : KS / 16;
#pragma unroll 4
        for (int k4 = 0; k4 < kSteps; k4++) {
            const float bv = ws[wrow][kb + 4 * k4];
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                acc[mt] = __builtin_amdgcn_mfma_f32_16x16x4f32(xs[16 * mt + col][kb + 4 * k4], bv, acc[mt], 0, 0, 0);
        }
    }
    // D layout: lane holds column lane & 15, rows 4 (lane >> 4) + r.
    if constexpr (NT == 4) {
        const int n = n0 + 16 * wave + (lane & 15);
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * mt + 4 * (lane >> 4) + r;
                if (m < M && n < N) Y[(int64_t)m * N + n] = acc[mt][r];
            }
    } else {
#pragma unroll
        for (int mt = 0; mt < MT; mt++) red[wave][mt][lane] = acc[mt];
        __syncthreads();
        for (int o = tid; o < MT * 64; o += 256) {  // the wave sums in wave order
            const int mt = o >> 6, ln = o & 63;
            const f32x4 v = ((red[0][mt][ln] + red[1][mt][ln]) + red[2][mt][ln]) + red[3][mt][ln];
            const int n = n0 + (ln & 15);
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int m = m0 + 16 * mt + 4 * (ln >> 4) + r;
                if (m < M && n < N) Y[(int64_t)m * N + n] = v[r];
            }
        }
    }
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

size_t gemm_workspace_bytes(int type_id, int M, int N, int K) {
    if (type_id == kQ8_0 && M <= 32) return 0;  // the skinny kernel
    return gemm_tile_workspace_bytes(type_id, M, N, K);
}

// The need peaks at multiples of the 128-row tile and is zero once the tiles
// cover the CUs; the splits keep (S - 1) tiles' partials per tile, below
// cu_count 128 x 128 floats (16 MiB on 256 CUs).
size_t gemm_workspace_max_bytes(int type_id, int N, int K) {
    size_t most = 0;
    for (int mt = 1; mt <= 64; mt++) {
        const size_t b = gemm_workspace_bytes(type_id, 128 * mt, N, K);
        if (b > most) most = b;
    }
    return most;
}

hipError_t launch_gemm_bf16(int type_id, const uint8_t *w, int64_t row_bytes, const uint16_t *x, float *y,
                            int M, int N, int K, hipStream_t stream, float *workspace, size_t workspace_bytes,
                            const uint8_t *prep, int64_t prep_rows) {
    if (M <= 0) return hipSuccess;
    const bool aligned = (reinterpret_cast<uintptr_t>(w) & 3u) == 0 && (row_bytes & 3) == 0 &&
                         (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    // M <= 4: the GEMV's column kernel, two vectors in each MFMA (on the
    // prepared column layout when there is one for its partition).
    if (gemm_col_supported(type_id, row_bytes, M, N, K, w != nullptr ? w : prep, x))
        return launch_gemm_col(type_id, w, row_bytes, x, y, M, N, K, stream, prep, prep_rows);
    if (w == nullptr) return hipErrorInvalidValue;  // the GGUF rows are needed
    // M <= 32 with Q8_0 weights: the buffer->LDS ring over 16-row column tiles.
    if (type_id == kQ8_0 && aligned && M <= 32 && N % 16 == 0 && K % 256 == 0 &&
        (int64_t)16 * row_bytes < ((int64_t)1 << 31) && (int64_t)M * K * 2 < ((int64_t)1 << 31)) {
        if (M <= 16)
            hipLaunchKernelGGL((gemm_q8_0_bf16_skinny_kernel<1, 4>), dim3(N / 16), dim3(256), 0, stream, w,
                               row_bytes, x, y, M, N, K);
        else
            hipLaunchKernelGGL((gemm_q8_0_bf16_skinny_kernel<2, 4>), dim3(N / 16), dim3(256), 0, stream, w,
                               row_bytes, x, y, M, N, K);
        return hipGetLastError();
    }
    // 128 x 128 tiles for Q8_0, Q4_0 and Q4_K (K a multiple of 256).
    if (gemm_tile_supported(type_id, row_bytes, M, N, K, w, x, y))
        return launch_gemm_tile(type_id, w, row_bytes, x, y, M, N, K, stream, workspace, workspace_bytes);
    // Other shapes and alignments.
    if (type_id == kQ8_0 && aligned) {
        if (M <= 16 && N % 16 == 0 && K % 256 == 0)
            return launch_tiled<16, 16, 16, 16, 4>(w, row_bytes, x, y, M, N, K, stream);
        if (M <= 128 && N % 16 == 0 && K % 64 == 0)
            return launch_tiled<128, 16, 32, 16, 1>(w, row_bytes, x, y, M, N, K, stream);
        if (N % 64 == 0 && K % 64 == 0)
            return launch_tiled<128, 64, 64, 32, 1>(w, row_bytes, x, y, M, N, K, stream);
    }
    // Q6_K with 4-byte aligned X rows: the fp32 matrix-core kernel, tiles of
    // 16 W rows and 16 / 32 / 64 X rows, or 64 x 64 tiles when those still
    // give every CU two workgroups (fewer re-reads of X).
    if (type_id == kQ6_K && K % kQK == 0 && (reinterpret_cast<uintptr_t>(x) & 3u) == 0 &&
        ((reinterpret_cast<uintptr_t>(w) | (uintptr_t)row_bytes) & 1u) == 0) {
        const int mt = M <= 16 ? 1 : M <= 32 ? 2 : 4;
        const int64_t wide = (int64_t)((N + 63) / 64) * ((M + 63) / 64);
        if (mt == 4 && wide >= 2 * (int64_t)device_cus()) {
            const dim3 g6((unsigned)((N + 63) / 64), (unsigned)((M + 63) / 64));
            hipLaunchKernelGGL((gemm_q6k_f32_kernel<4, 4>), g6, dim3(256), 0, stream, w, row_bytes, x, y, M, N, K);
        } else {
            const dim3 g6((unsigned)((N + 15) / 16), (unsigned)((M + 16 * mt - 1) / (16 * mt)));
            if (mt == 1)
                hipLaunchKernelGGL((gemm_q6k_f32_kernel<1, 1>), g6, dim3(256), 0, stream, w, row_bytes, x, y, M, N, K);
            else if (mt == 2)
                hipLaunchKernelGGL((gemm_q6k_f32_kernel<2, 1>), g6, dim3(256), 0, stream, w, row_bytes, x, y, M, N, K);
            else
                hipLaunchKernelGGL((gemm_q6k_f32_kernel<4, 1>), g6, dim3(256), 0, stream, w, row_bytes, x, y, M, N, K);
        }
        return hipGetLastError();
    }
    if (type_id == kQ5_K || type_id == kQ6_K) {
        const dim3 g16((unsigned)((N + 15) / 16), (unsigned)((M + 15) / 16));
        if (type_id == kQ5_K)
            hipLaunchKernelGGL(gemm_kquant_generic_kernel<kQ5_K>, g16, dim3(256), 0, stream, w, row_bytes, x, y, M,
                               N, K);
        else
            hipLaunchKernelGGL(gemm_kquant_generic_kernel<kQ6_K>, g16, dim3(256), 0, stream, w, row_bytes, x, y, M,
                               N, K);
        return hipGetLastError();
    }
    const int64_t total = (int64_t)M * N;
    const dim3 grid((unsigned)((total + 255) / 256)), block(256);
    switch (type_id) {
    case kQ8_0:
        hipLaunchKernelGGL(gemm_q8_0_generic_kernel, grid, block, 0, stream, w, row_bytes, x, y, M, N, K);
        break;
    case kQ4_0:
        hipLaunchKernelGGL(gemm_generic_kernel<kQ4_0>, grid, block, 0, stream, w, row_bytes, x, y, M, N, K);
        break;
    case kQ4_K:
        hipLaunchKernelGGL(gemm_generic_kernel<kQ4_K>, grid, block, 0, stream, w, row_bytes, x, y, M, N, K);
        break;
    default:
        return hipErrorInvalidValue;
    }
    return hipGetLastError();
}

}  // namespace gollek
