// gguf_gemm_tile.hip -- small-M GEMM (prefill / batched decode) Y = X . W^T
// for Q8_0, Q4_0 and Q4_K weights on gfx950 bf16 MFMA, fp32 accumulate.
//
// Y[M, N] = X[M, K] . W[N, K]^T with X bf16 (row-major M x K) and W the GGUF
// matrix (N rows of K columns), the Linear convention of
// runner/safetensor/gollek-safetensor-core/src/main/java/tech/kayys/gollek/
// safetensor/core/tensor/AccelOps.java:370-376.  The reference has no GGUF
// GEMM: its prefill runs M independent raw mat-vecs per weight
// (RT/GgufTensorOps.java:666-674; RT/ = runner/gguf/gollek-gguf-core/src/
// main/java/tech/kayys/gollek/gguf/runtime/), each summing per block
// d * sum(q * x) (RT/GgufQ8RawDot.java:137-184, RT/GgufQ32RawDot.java:33-66)
// or, for Q4_K, per 32-element sub-block fl(d*sc) * sum(q * x) - fl(dmin*m)
// * sum(x) (RT/GgufQ4RawDot.java:331-674).
//
// Exactness.  Each v_mfma_f32_16x16x32_bf16 contracts one 32-element block
// (or Q4_K sub-block) of X with the block's integer codes, which bf16 holds
// exactly (Q8_0 q in [-127, 127], Q4_0 q - 8 in [-8, 7]; Q4_K as 128 + q,
// q in [0, 15]); the block's fp32 scale is applied to that fp32 result in
// one FMA per output, the reference's block structure.  The Q4_K min term
// needs sum(x) over the sub-block per X row: one more MFMA per 16-row tile
// with an all-ones B operand puts it in the same lanes as the products, and
// a second FMA subtracts (dmin * m + 128 * d) times it, which also removes
// the codes' offset of 128 (dmin * m is 0 when the min code is 0, so a
// non-finite dmin stays out as in RT/GgufKQuantLayout.java:67-69).  The
// offset makes the fp32 sums run at ~128 |x| instead of ~8 |x|: about 2^-17
// of sum |x| of absolute error per sub-block, far inside the 1e-2 bar, and a
// non-finite d gives NaN rather than +-inf.
//
// Tiling.  A workgroup owns a 128 x 128 tile of Y: 8 compute waves and 2
// loader waves.  K advances in stages of 64 columns (two blocks).  Compute
// wave w contracts block w / 4 of the stage for all 128 rows of X and
// columns 32 (w % 4) .. 32 (w % 4) + 31 of the tile, and the two blocks'
// tiles are added at the end (first-block sum + second-block sum).  The
// loader waves move each stage's X (128 rows x 128 bytes) and the W rows' raw
// bytes for the stage by buffer->LDS loads into a ring of slots, several
// stages ahead; the compute waves issue no global loads, so they never stall
// on a full queue of outstanding loads.  Each compute wave widens its own
// columns' codes from the raw bytes to bf16 in registers (B operand) with
// their fp32 block scales, so no converted copy passes through LDS; its LDS
// reads of a stage are issued together (raw codes first) and waited for in
// order, so the MFMAs of row tile i start when tile i has arrived.  One
// barrier per stage.  The tile leaves through LDS as whole rows, stored 16
// bytes a lane with nontemporal stores.
//
// Split-K.  When the tiles alone leave CUs idle (M = 512 at N = 4096: 128
// tiles on 256 CUs), each tile's K range is split over S workgroups: split 0
// writes Y, split k > 0 a partial tile in the workspace, and a second kernel
// adds the partials to Y in split order, so the result does not depend on
// timing.  Per CU this halves (S = 2) the X and W bytes a 128 x 64 tile over
// the whole of K would take in from L2, which is what bounds these shapes.
// (Adding two splits' partials inside the kernel instead, the second
// workgroup of a tile to finish reading the first's partial after an
// agent-scope release / acquire, measured 54 us against 35 us at M = 512:
// the release writes back and the acquire invalidates each XCD's L2.)
#include "gguf_blocks.hpp"
#include "gguf_dot4.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

constexpr int kTileMMax = 128, kTileN = 128;  // a tile is 16 MT x 128, MT = 1, 2, 4 or 8
constexpr int kRowB = 128;                     // LDS bytes per X row per stage (64 bf16)
constexpr int kThreads = 640;                  // 8 compute waves + 2 loader waves
constexpr int kCompute = 512;
constexpr int kStagePitch = kTileN + 4;        // floats per row of the output staging

// Raw W bytes of one row for one stage (64 columns), moved as kChunks
// 16-byte chunks that land contiguously in LDS (row pitch 16 kChunks bytes):
//   Q8_0: the row's two 34-byte blocks (68 bytes; 5 chunks, the last 12
//         bytes belong to the next stage and are not used)
//   Q4_0: two 18-byte blocks (36 bytes; 3 chunks, 12 unused)
//   Q4_K: the superblock header (16 bytes: d, dmin, 12 scale bytes) and the
//         32 quant bytes of the stage's chunk c (sub-blocks 2c, 2c + 1)
//   Q5_K: the header, the superblock's 32 qh bytes (bits 2c, 2c + 1 are the
//         chunk's fifth bits) and the chunk's 32 quant bytes (80 bytes)
//   Q6_K: the chunk's half (h = c >> 1) of ql (64 bytes) and of qh (32)
//         from 0 or 2 bytes before them (m: superblocks of odd index begin 2
//         bytes past a dword), and 32 bytes holding the scales and d (bytes
//         192 .. 209) from byte 192 (m = 0) or 178 (m = 2): 5 + 3 + 2 chunks
//         (160 bytes).  Rows of an even superblock count end with an odd
//         superblock, so no load runs past a row's end; an even superblock's
//         last chunk reads 14 bytes of the next one.
template <int T>
struct RawW;
template <>
struct RawW<kQ8_0> {
    static constexpr int kChunks = 5, kStageBytes = 68, kSlots = 5;
};
template <>
struct RawW<kQ4_0> {
    static constexpr int kChunks = 3, kStageBytes = 36, kSlots = 6;
};
template <>
struct RawW<kQ4_K> {
    static constexpr int kChunks = 3, kStageBytes = 0, kSlots = 6;  // 144 bytes per four stages
};
template <>
struct RawW<kQ5_K> {
    static constexpr int kChunks = 5, kStageBytes = 0, kSlots = 6;  // 176 bytes per four stages
};
template <>
struct RawW<kQ6_K> {
    static constexpr int kChunks = 10, kStageBytes = 0, kSlots = 4;  // 210 bytes per four stages
};

// Geometry of a 16 MT x 128 tile: MT row tiles of 16 rows of X.  Tiles of
// fewer rows (small M) are load-latency bound and use the LDS they leave free
// for a deeper ring, as deep as the loader waves' vmcnt waits can count.
template <int T, int MT>
struct TileGeom {
    static constexpr int kTileM = 16 * MT;
    static constexpr int kXBytes = kTileM * kRowB;  // X of a stage
    static constexpr int kPitch = 16 * RawW<T>::kChunks;
    static constexpr int kRawBytes = kTileN * kPitch;
    static constexpr int kSlot = kXBytes + kRawBytes;
    static constexpr int kInstr = kTileN * RawW<T>::kChunks / 64;  // 16-byte W DMA instructions
    static_assert(kInstr % 2 == 0, "W loads split evenly over the two loader waves");
    static constexpr int kLoads = MT + kInstr / 2;                 // loads per loader wave per stage
    static constexpr int kDeep = (160 * 1024 / kSlot) < (63 / kLoads + 2) ? (160 * 1024 / kSlot) : (63 / kLoads + 2);
    static constexpr int kSlots = MT == 8 ? RawW<T>::kSlots : (kDeep < 8 ? kDeep : 8);
    static constexpr int kRing = kSlots * kSlot;
    static constexpr bool kMins = T == kQ4_K || T == kQ5_K;
    static_assert(kRing <= 160 * 1024, "LDS budget");
    static_assert(kLoads * (kSlots - 2) <= 63, "vmcnt range of the loader waits");
    static_assert(kRing >= 4 * MT * 2 * 1024 && kRing >= kTileM * kStagePitch * 4, "epilogue staging");
};

__device__ __forceinline__ uint32_t swz(int r, int kc) {
    return (uint32_t)(r * kRowB + 16 * (kc ^ ((r >> 1) & 7)));
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    // Exact for the integer codes here (|v| <= 128).
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, bf16x2));
}

// Four signed bytes -> two dwords of bf16 pairs (v_cvt_f32_i32 with a
// sign-extended byte select each, then v_cvt_pk_bf16_f32).
__device__ __forceinline__ void s8x4_bf16(uint32_t w, uint32_t &a, uint32_t &b) {
    a = pack_bf16x2((float)(int)(int8_t)(w & 0xFFu), (float)(int)(int8_t)((w >> 8) & 0xFFu));
    b = pack_bf16x2((float)(int)(int8_t)((w >> 16) & 0xFFu), (float)(int)(int8_t)(w >> 24));
}

// Four 4-bit codes q (one per byte of w) -> two dwords of bf16 pairs
// holding 128 + q exactly: the bf16 bit pattern 0x4300 | q is 128 + q (at
// 128 a bf16 step is 1), so one byte permute per pair instead of two
// conversions.
__device__ __forceinline__ void q4x4_bf16_128(uint32_t w, uint32_t &a, uint32_t &b) {
    a = __builtin_amdgcn_perm(0x43434343u, w, 0x04010400u);  // {w.b0, 0x43, w.b1, 0x43}
    b = __builtin_amdgcn_perm(0x43434343u, w, 0x04030402u);  // {w.b2, 0x43, w.b3, 0x43}
}

// 16-byte buffer->LDS load (a plain __device__ function: the builtin used
// directly in a kernel template's body drops hipcc's host launch stub).
__device__ __forceinline__ void dma16(__amdgpu_buffer_rsrc_t rs, void *dst, uint32_t off) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)dst, 16, off, 0, 0, 0);
}

// Stage barriers (compiler memory barriers too): a loader wave first waits
// until all but its last N loads have landed, a compute wave until its LDS
// accesses are done.
template <int N>
__device__ __forceinline__ void loader_barrier() {
    asm volatile("s_waitcnt vmcnt(%0)\n\ts_barrier" : : "n"(N) : "memory");
}
// loader_barrier<KL * later> for a wave-uniform 0 <= later <= L.
template <int KL, int L>
__device__ __forceinline__ void loader_barrier_n(int later) {
    if constexpr (L == 0) {
        loader_barrier<0>();
    } else {
        if (later >= L) loader_barrier<KL * L>();
        else loader_barrier_n<KL, L - 1>(later);
    }
}
__device__ __forceinline__ void compute_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ f32x4 mfma_bf16(bf16x8 a, bf16x8 b) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, f32x4{0.0f, 0.0f, 0.0f, 0.0f}, 0, 0, 0);
}

// Every LDS access inside the stage loop is inline asm: the compiler cannot
// tell which buffer->LDS load filled which bytes and would otherwise wait for
// every load in flight before each LDS access.  The explicit vmcnt wait and
// barrier of each stage make the data visible; a wave's reads of a stage are
// issued by one statement and its registers named by the lgkmcnt wait that
// follows, so that no use is scheduled before the data has arrived.
//
// One stage's operands of a wave: per column tile i (rows 16 apart: +RP
// bytes) the raw code dwords (q0..q2 at b; Q4_K: q0, q1) and the scale dword
// (at s; Q4_K: the 16-byte header), then A (MT row tiles of X, at a +
// 2048 i), each read by its own statement in that order (volatile asm keeps
// the order).  LDS reads complete in order, so the raw codes can be widened
// once ops_wait_raw returns while the A tiles still arrive, and row tile i
// waits only for its own data (ops_wait_a).
struct Ops {
    u32x4 a[8];
    uint32_t q[2][3], sc[2];  // Q8_0, Q4_0
    uint2 q2[2];              // Q4_K, Q5_K
    u32x4 hd[2];              // Q4_K, Q5_K
    uint2 qh[2];              // Q5_K
    uint32_t l6[2][3], h6[2][3], d6[2];  // Q6_K: ql, qh dwords, d
    uint32_t s6[2][2];                   // Q6_K: scale bytes
};
template <int RP>
__device__ __forceinline__ void ops_read_q32(uint32_t b, uint32_t s, Ops &o) {
    asm volatile(
        "ds_read_b32 %0, %8\n\t"
        "ds_read_b32 %1, %8 offset:4\n\t"
        "ds_read_b32 %2, %8 offset:8\n\t"
        "ds_read_b32 %3, %9\n\t"
        "ds_read_b32 %4, %8 offset:%10\n\t"
        "ds_read_b32 %5, %8 offset:%11\n\t"
        "ds_read_b32 %6, %8 offset:%12\n\t"
        "ds_read_b32 %7, %9 offset:%10"
        : "=&v"(o.q[0][0]), "=&v"(o.q[0][1]), "=&v"(o.q[0][2]), "=&v"(o.sc[0]), "=&v"(o.q[1][0]),
          "=&v"(o.q[1][1]), "=&v"(o.q[1][2]), "=&v"(o.sc[1])
        : "v"(b), "v"(s), "n"(RP), "n"(RP + 4), "n"(RP + 8)
        : "memory");
}
template <int RP>
__device__ __forceinline__ void ops_read_q4k(uint32_t b, uint32_t s, Ops &o) {
    asm volatile(
        "ds_read_b64 %0, %4\n\t"
        "ds_read_b128 %1, %5\n\t"
        "ds_read_b64 %2, %4 offset:%6\n\t"
        "ds_read_b128 %3, %5 offset:%6"
        : "=&v"(o.q2[0]), "=&v"(o.hd[0]), "=&v"(o.q2[1]), "=&v"(o.hd[1])
        : "v"(b), "v"(s), "n"(RP)
        : "memory");
}
// Q5_K: ops_read_q4k plus the lane's 8 qh bytes of each column tile (at h).
template <int RP>
__device__ __forceinline__ void ops_read_q5k(uint32_t b, uint32_t s, uint32_t h, Ops &o) {
    asm volatile(
        "ds_read_b64 %0, %6\n\t"
        "ds_read_b64 %1, %8\n\t"
        "ds_read_b128 %2, %7\n\t"
        "ds_read_b64 %3, %6 offset:%9\n\t"
        "ds_read_b64 %4, %8 offset:%9\n\t"
        "ds_read_b128 %5, %7 offset:%9"
        : "=&v"(o.q2[0]), "=&v"(o.qh[0]), "=&v"(o.hd[0]), "=&v"(o.q2[1]), "=&v"(o.qh[1]), "=&v"(o.hd[1])
        : "v"(b), "v"(s), "v"(h), "n"(RP)
        : "memory");
}
// Q6_K: per column tile the lane's 3 ql dwords (at l), 3 qh dwords (at h),
// the 2 dwords of scale bytes from s and the dword holding d (at dd).
template <int RP>
__device__ __forceinline__ void ops_read_q6k(uint32_t l, uint32_t h, uint32_t s, uint32_t dd, Ops &o) {
    asm volatile(
        "ds_read_b32 %0, %18\n\t"
        "ds_read_b32 %1, %18 offset:4\n\t"
        "ds_read_b32 %2, %18 offset:8\n\t"
        "ds_read_b32 %3, %19\n\t"
        "ds_read_b32 %4, %19 offset:4\n\t"
        "ds_read_b32 %5, %19 offset:8\n\t"
        "ds_read_b32 %6, %20\n\t"
        "ds_read_b32 %7, %20 offset:4\n\t"
        "ds_read_b32 %8, %21\n\t"
        "ds_read_b32 %9, %18 offset:%22\n\t"
        "ds_read_b32 %10, %18 offset:%23\n\t"
        "ds_read_b32 %11, %18 offset:%24\n\t"
        "ds_read_b32 %12, %19 offset:%22\n\t"
        "ds_read_b32 %13, %19 offset:%23\n\t"
        "ds_read_b32 %14, %19 offset:%24\n\t"
        "ds_read_b32 %15, %20 offset:%22\n\t"
        "ds_read_b32 %16, %20 offset:%23\n\t"
        "ds_read_b32 %17, %21 offset:%22"
        : "=&v"(o.l6[0][0]), "=&v"(o.l6[0][1]), "=&v"(o.l6[0][2]), "=&v"(o.h6[0][0]), "=&v"(o.h6[0][1]),
          "=&v"(o.h6[0][2]), "=&v"(o.s6[0][0]), "=&v"(o.s6[0][1]), "=&v"(o.d6[0]), "=&v"(o.l6[1][0]),
          "=&v"(o.l6[1][1]), "=&v"(o.l6[1][2]), "=&v"(o.h6[1][0]), "=&v"(o.h6[1][1]), "=&v"(o.h6[1][2]),
          "=&v"(o.s6[1][0]), "=&v"(o.s6[1][1]), "=&v"(o.d6[1])
        : "v"(l), "v"(h), "v"(s), "v"(dd), "n"(RP), "n"(RP + 4), "n"(RP + 8)
        : "memory");
}
template <int I>
__device__ __forceinline__ void ops_read_a(uint32_t a, Ops &o) {
    asm volatile("ds_read_b128 %0, %1 offset:%2" : "=&v"(o.a[I]) : "v"(a), "n"(2048 * I) : "memory");
}
// Row tiles 0 .. MT - 1, in order.
template <int MT>
__device__ __forceinline__ void ops_read_as(uint32_t a, Ops &o) {
    ops_read_a<0>(a, o);
    if constexpr (MT > 1) ops_read_a<1>(a, o);
    if constexpr (MT > 2) {
        ops_read_a<2>(a, o);
        ops_read_a<3>(a, o);
    }
    if constexpr (MT > 4) {
        ops_read_a<4>(a, o);
        ops_read_a<5>(a, o);
        ops_read_a<6>(a, o);
        ops_read_a<7>(a, o);
    }
}
// The raw dwords have arrived (the MT A reads may still be outstanding).
template <int MT>
__device__ __forceinline__ void ops_wait_raw(Ops &o) {
    asm volatile("s_waitcnt lgkmcnt(%14)"
                 : "+v"(o.q[0][0]), "+v"(o.q[0][1]), "+v"(o.q[0][2]), "+v"(o.sc[0]), "+v"(o.q[1][0]),
                   "+v"(o.q[1][1]), "+v"(o.q[1][2]), "+v"(o.sc[1]), "+v"(o.q2[0]), "+v"(o.q2[1]),
                   "+v"(o.hd[0]), "+v"(o.hd[1]), "+v"(o.qh[0]), "+v"(o.qh[1])
                 : "n"(MT)
                 : "memory");
}
// Q6_K: the same wait for its raw dwords.
template <int MT>
__device__ __forceinline__ void ops_wait_raw6(Ops &o) {
    asm volatile("s_waitcnt lgkmcnt(%18)"
                 : "+v"(o.l6[0][0]), "+v"(o.l6[0][1]), "+v"(o.l6[0][2]), "+v"(o.h6[0][0]), "+v"(o.h6[0][1]),
                   "+v"(o.h6[0][2]), "+v"(o.s6[0][0]), "+v"(o.s6[0][1]), "+v"(o.d6[0]), "+v"(o.l6[1][0]),
                   "+v"(o.l6[1][1]), "+v"(o.l6[1][2]), "+v"(o.h6[1][0]), "+v"(o.h6[1][1]), "+v"(o.h6[1][2]),
                   "+v"(o.s6[1][0]), "+v"(o.s6[1][1]), "+v"(o.d6[1])
                 : "n"(MT)
                 : "memory");
}
// Row tile I has arrived (the MT - 1 - I later ones may still be outstanding).
template <int MT, int I>
__device__ __forceinline__ void ops_wait_a(Ops &o) {
    asm volatile("s_waitcnt lgkmcnt(%1)" : "+v"(o.a[I]) : "n"(MT - 1 - I) : "memory");
}
// ops_wait_a for row tile i (a constant after unrolling).
template <int MT>
__device__ __forceinline__ void ops_wait_row(int i, Ops &o) {
    if (i == 0) ops_wait_a<MT, 0>(o);
    if constexpr (MT > 1)
        if (i == 1) ops_wait_a<MT, 1>(o);
    if constexpr (MT > 2) {
        if (i == 2) ops_wait_a<MT, 2>(o);
        if (i == 3) ops_wait_a<MT, 3>(o);
    }
    if constexpr (MT > 4) {
        if (i == 4) ops_wait_a<MT, 4>(o);
        if (i == 5) ops_wait_a<MT, 5>(o);
        if (i == 6) ops_wait_a<MT, 6>(o);
        if (i == 7) ops_wait_a<MT, 7>(o);
    }
}

}  // namespace

// One 16 MT x 128 tile of Y (or of split `split`'s partial sum) per workgroup.
template <int T, int MT>
__global__ __launch_bounds__(kThreads) void gemm_tile_kernel(const uint8_t *__restrict__ W,
                                                            int64_t row_bytes,
                                                            const uint16_t *__restrict__ X,
                                                            float *__restrict__ Y, int M, int N,
                                                            int K, int S, float *__restrict__ part) {
    using G = TileGeom<T, MT>;
    using R = RawW<T>;
    constexpr int NS = G::kSlots;
    constexpr int kTileM = G::kTileM, kXBytes = G::kXBytes;
    // The ring: X and raw W of NS stages; at the end the output staging.
    __shared__ __attribute__((aligned(16))) uint8_t ring[G::kRing];

    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);

    // Tile order: the splits outermost; inside a split, groups of up to four
    // M tiles with the N tiles N-major inside a group, so that the 32
    // workgroups an XCD runs (workgroups are dealt to the 8 XCDs round robin;
    // v renumbers them XCD-major) share X and W rows in that XCD's L2.
    const int tm = (M + kTileM - 1) / kTileM, tn = (N + kTileN - 1) / kTileN;
    const int G8 = (int)gridDim.x;
    const int v = (G8 % 8 == 0) ? (int)(blockIdx.x % 8) * (G8 / 8) + (int)(blockIdx.x / 8) : (int)blockIdx.x;
    const int split = v / (tm * tn);
    const int t = v - split * tm * tn;
    const int grp = t / (4 * tn);
    const int first_m = 4 * grp;
    const int gm = tm - first_m < 4 ? tm - first_m : 4;
    const int local = t - grp * 4 * tn;
    const int m0 = (first_m + local % gm) * kTileM, n0 = (local / gm) * kTileN;
    const int nst = K / 64 / S;  // stages of this split (a multiple of 4)
    const int s0 = split * nst;

    // Buffers from the split's first column; rows past M / N and bytes past
    // the end read as zeros.
    const int mrows = M - m0 < kTileM ? M - m0 : kTileM;
    const int nrows = N - n0 < kTileN ? N - n0 : kTileN;
    // (Q6_K: none; its loads start up to 2 bytes before a superblock, so the
    // offsets stay relative to the rows' first byte)
    const int64_t w_split = T == kQ4_K   ? (int64_t)(s0 / 4) * 144
                            : T == kQ5_K ? (int64_t)(s0 / 4) * kQ5KBlockBytes
                            : T == kQ6_K ? 0
                                         : (int64_t)s0 * R::kStageBytes;
    const __amdgpu_buffer_rsrc_t xr = wave_buffer(
        reinterpret_cast<const uint8_t *>(X) + (int64_t)m0 * K * 2 + (int64_t)s0 * 128,
        (uint32_t)((int64_t)mrows * K * 2 - (int64_t)s0 * 128));
    const __amdgpu_buffer_rsrc_t wr = wave_buffer(W + (int64_t)n0 * row_bytes + w_split,
                                                  (uint32_t)((int64_t)nrows * row_bytes - w_split));

    // ---- loads of a stage (loader waves 8 and 9) ---------------------------
    // X: loader l moves LDS chunks p = 64 (MT l + i) + lane (i < MT): row p / 8
    // at swizzled position p % 8, holding the row's column chunk
    // position ^ ((row >> 1) & 7).  W: instruction j moves lane-chunks q =
    // 64 j + lane (row q / kChunks, part q % kChunks) to LDS offset 16 q;
    // loader l takes instructions l, l + 2, ...  Q4_K: part 0 is the header,
    // parts 1 and 2 the quants at 16 + 32 c + 16 (part - 1).
    const int ldr = wave - 8;
    auto issue = [&](int ls) {
        uint8_t *const xs = ring + (ls % NS) * G::kSlot;
        uint8_t *const rs = xs + kXBytes;
#pragma unroll
        for (int i = 0; i < MT; i++) {
            const int p = 64 * (MT * ldr + i) + lane;
            const int r = p >> 3, kc = (p & 7) ^ ((r >> 1) & 7);
            dma16(xr, xs + 1024 * (MT * ldr + i),
                  (uint32_t)r * (uint32_t)(2 * K) + 16u * (uint32_t)kc + 128u * (uint32_t)ls);
        }
#pragma unroll
        for (int i = 0; i < G::kInstr / 2; i++) {
            const int j = ldr + 2 * i;
            const int q = 64 * j + lane;
            const int row = q / R::kChunks, part = q - row * R::kChunks;
            uint32_t off = (uint32_t)row * (uint32_t)row_bytes + (uint32_t)(16 * part);
            if constexpr (T == kQ4_K)
                off += (uint32_t)(144 * (ls >> 2)) + (part != 0 ? (uint32_t)(32 * (ls & 3)) : 0u);
            else if constexpr (T == kQ5_K)  // parts 0..2: header, qh; 3, 4: the chunk's quants at 48
                off += (uint32_t)(kQ5KBlockBytes * (ls >> 2)) + (part >= 3 ? (uint32_t)(32 * (ls & 3)) : 0u);
            else if constexpr (T == kQ6_K) {
                // superblock sb from its dword at or before it (m = 2 (sb & 1)); parts
                // 0..4: ql half h from 64 h, 5..7: qh half h from 128 + 32 h (both
                // less m), 8, 9: from 192 (m = 0) or 178 (m = 2)
                const int sb = (s0 >> 2) + (ls >> 2), h = (ls >> 1) & 1, m2 = sb & 1;
                const int at = part < 5 ? 64 * h + 16 * part
                               : part < 8 ? 128 + 32 * h + 16 * (part - 5)
                                          : (m2 ? 180 : 192) + 16 * (part - 8);
                off = (uint32_t)row * (uint32_t)row_bytes + (uint32_t)(210 * sb - 2 * (sb & 1) + at);
            } else
                off += (uint32_t)(R::kStageBytes * ls);
            dma16(wr, rs + 1024 * j, off);
        }
    };

    // ---- a wave's operands -----------------------------------------------
    // Wave w: block kg = w / 4 of each stage, tile columns 32 nq .. 32 nq + 31
    // (nq = w % 4) in two 16-column tiles, all 16 MT rows in MT 16-row tiles.
    // Lane: A row (and B column) lane & 15, k group lk = lane >> 4 (k 8 lk ..
    // 8 lk + 7 of the block).
    const int kg = wave >> 2, nq = wave & 3;
    const int lr = lane & 15, lk = lane >> 4;
    const uint32_t ring_base = (uint32_t)(uintptr_t)(lds_ptr)ring;
    const uint32_t xa = ring_base + swz(lr, 4 * kg + lk);
    const uint32_t wrow = ring_base + (uint32_t)(kXBytes + G::kPitch * (32 * nq + lr));
    // Per-lane code and scale offsets in a row's raw bytes, and the byte shift
    // that realigns the codes.
    uint32_t qoff, soff, qsh, nsh;
    if constexpr (T == kQ8_0) {
        // block kg's 8 codes of lane group lk at byte 2 + 34 kg + 8 lk; scale in dword 8 kg
        qoff = (uint32_t)(4 * (kg ? 9 + 2 * lk : 2 * lk));
        qsh = kg ? 0u : 2u;
        soff = (uint32_t)(32 * kg);
        nsh = 16u * (uint32_t)kg;  // scale half
    } else if constexpr (T == kQ4_0) {
        // 8 bytes of block kg at byte 2 + 18 kg + 8 (lk & 1); nibble lk >> 1; scale in dword 4 kg
        qoff = (uint32_t)(4 * (kg ? 5 + 2 * (lk & 1) : 2 * (lk & 1)));
        qsh = kg ? 0u : 2u;
        soff = (uint32_t)(16 * kg);
        nsh = 16u * (uint32_t)kg;
    } else {
        // quant bytes 8 lk .. 8 lk + 7 of the chunk at 16 + 8 lk (Q5_K: at
        // 48 + 8 lk, its qh bytes 8 lk .. 8 lk + 7 at 16 + 8 lk); header at 0
        qoff = (uint32_t)((T == kQ5_K ? 48 : 16) + 8 * lk);
        qsh = 0u;
        soff = 0u;
        nsh = 0u;
    }
    const uint32_t qhoff = (uint32_t)(16 + 8 * lk);       // Q5_K
    const int nib = T == kQ4_0 ? 4 * (lk >> 1) : 4 * kg;  // nibble shift (Q4_0, Q4_K, Q5_K)

    f32x4 acc[MT][2];
#pragma unroll
    for (int a = 0; a < MT; a++)
#pragma unroll
        for (int b = 0; b < 2; b++) acc[a][b] = f32x4{0.0f, 0.0f, 0.0f, 0.0f};
    const bf16x8 ones = __builtin_bit_cast(bf16x8, u32x4{0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u});

    // Per stage: 2 MT MFMAs (MT row tiles x 2 column tiles; Q4_K: one more
    // per row tile for the sums of x) and one FMA (Q4_K: two) per output.
    // The FMAs of each MFMA are issued two MFMAs later, so that no FMA waits
    // for the MFMA it consumes.
    auto compute = [&](int ls) {
        const uint32_t so = (uint32_t)((ls % NS) * G::kSlot);
        Ops o;
        if constexpr (T == kQ4_K)
            ops_read_q4k<16 * G::kPitch>(wrow + so + qoff, wrow + so + soff, o);
        else if constexpr (T == kQ5_K)
            ops_read_q5k<16 * G::kPitch>(wrow + so + qoff, wrow + so + soff, wrow + so + qhoff, o);
        else
            ops_read_q32<16 * G::kPitch>(wrow + so + qoff, wrow + so + soff, o);
        ops_read_as<MT>(xa + so, o);
        ops_wait_raw<MT>(o);
        bf16x8 B[2];
        float d[2], dm[2];
        // Column tile i's codes as bf16 (B operand) and its scale / min term.
        auto widen = [&](int i) {
            uint32_t c[4];
            if constexpr (T == kQ8_0) {
                const uint32_t w0 = __builtin_amdgcn_alignbyte(o.q[i][1], o.q[i][0], qsh);
                const uint32_t w1 = __builtin_amdgcn_alignbyte(o.q[i][2], o.q[i][1], qsh);
                s8x4_bf16(w0, c[0], c[1]);
                s8x4_bf16(w1, c[2], c[3]);
                d[i] = half_bits_to_float_fast(o.sc[i] >> nsh);
            } else if constexpr (T == kQ4_0) {
                // q - 8 as a signed byte: ((nib + 0x78) ^ 0x80)
                const uint32_t w0 = (__builtin_amdgcn_alignbyte(o.q[i][1], o.q[i][0], qsh) >> nib) & 0x0F0F0F0Fu;
                const uint32_t w1 = (__builtin_amdgcn_alignbyte(o.q[i][2], o.q[i][1], qsh) >> nib) & 0x0F0F0F0Fu;
                s8x4_bf16((w0 + 0x78787878u) ^ 0x80808080u, c[0], c[1]);
                s8x4_bf16((w1 + 0x78787878u) ^ 0x80808080u, c[2], c[3]);
                d[i] = half_bits_to_float_fast(o.sc[i] >> nsh);
            } else {
                // B holds 128 + q; the 128 sum(x) it adds comes off with the
                // min term: d (P - 128 sx) - dmin m sx = d P - (dmin m + 128 d) sx.
                // Q5_K: q's fifth bit is bit 2 c + kg of its qh byte (c = ls & 3).
                uint32_t lo = (o.q2[i].x >> nib) & 0x0F0F0F0Fu, hi = (o.q2[i].y >> nib) & 0x0F0F0F0Fu;
                if constexpr (T == kQ5_K) {
                    const int hb = 2 * (ls & 3) + kg;
                    lo |= ((o.qh[i].x >> hb) & 0x01010101u) << 4;
                    hi |= ((o.qh[i].y >> hb) & 0x01010101u) << 4;
                }
                q4x4_bf16_128(lo, c[0], c[1]);
                q4x4_bf16_128(hi, c[2], c[3]);
                uint32_t scp, mnp;
                q4k_pair_codes(o.hd[i].y, o.hd[i].z, o.hd[i].w, ls & 3, &scp, &mnp);
                const uint32_t scj = (scp >> (8 * kg)) & 0xFFu, mj = (mnp >> (8 * kg)) & 0xFFu;
                d[i] = half_bits_to_float_fast(o.hd[i].x & 0xFFFFu) * (float)scj;
                dm[i] = fmaf(128.0f, d[i], mj == 0u ? 0.0f : half_bits_to_float_fast(o.hd[i].x >> 16) * (float)mj);
            }
            B[i] = __builtin_bit_cast(bf16x8, u32x4{c[0], c[1], c[2], c[3]});
        };
        // MFMA k = 0 .. 2 MT - 1 is (row tile k % MT, column tile k / MT):
        // column tile 1 is widened while column tile 0's first MFMAs run, and
        // the FMAs of MFMA k - 2 are issued with MFMA k, so that none waits
        // for its MFMA.  Q4_K: the sums of x of row tile mt come with its
        // column-0 MFMA.
        f32x4 p[3], sx[MT];
        auto fmas = [&](int k) {
            const int mt = k % MT, nt = k / MT;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc[mt][nt][r] = fmaf(d[nt], p[k % 3][r], acc[mt][nt][r]);
                if constexpr (G::kMins) acc[mt][nt][r] = fmaf(-dm[nt], sx[mt][r], acc[mt][nt][r]);
            }
        };
        widen(0);
#pragma unroll
        for (int k = 0; k < 2 * MT + 2; k++) {
            __builtin_amdgcn_sched_barrier(0);
            if (k < 2 * MT) {
                const int mt = k % MT, nt = k / MT;
                if (k < MT) ops_wait_row<MT>(k, o);
                const bf16x8 A = __builtin_bit_cast(bf16x8, o.a[mt]);
                if (k == (MT < 2 ? MT : 2)) widen(1);
                if constexpr (G::kMins)
                    if (nt == 0) sx[mt] = mfma_bf16(A, ones);
                p[k % 3] = mfma_bf16(A, B[nt]);
            }
            if (k >= 2) fmas(k - 2);
        }
    };

    // Q6_K: a 32-column block holds two 16-element scale groups, so each
    // MFMA takes one group's codes (B_lo: lanes of k groups 0, 1; B_hi: 2, 3;
    // the other lanes zero) as 128 + q (q = ql nibble | qh bits << 4, 0..63),
    // starting from C = -160 sum(x) over the same lanes (an MFMA against a
    // constant -160 B), so its result is sum((q - 32) x) of the group; the
    // FMA applies fl(d sc) of the group (exact: an 11-bit d times an 8-bit
    // scale).  Per row tile two MFMAs for the starts and per column tile two
    // more, two FMAs per output.
    auto compute6 = [&](int ls) {
        const uint32_t so = (uint32_t)((ls % NS) * G::kSlot);
        const int c = ls & 3, m = 2 * (((s0 >> 2) + (ls >> 2)) & 1);
        const uint32_t rb = wrow + so;  // this lane's W row: ql piece, qh piece at 80, tail at 128
        Ops o;
        ops_read_q6k<16 * G::kPitch>(rb + 32 * kg + 8 * lk, rb + 80 + 8 * lk, rb + 128 + 4 * c + 6 * m,
                                     rb + 144 + 6 * m, o);
        ops_read_as<MT>(xa + so, o);
        ops_wait_raw6<MT>(o);
        const int nib = 4 * (c & 1), hsh = 2 * (2 * (c & 1) + kg);
        const bool lo_half = lk < 2;
        const u32x4 zero = {0u, 0u, 0u, 0u};
        const u32x4 m160 = {0xC320C320u, 0xC320C320u, 0xC320C320u, 0xC320C320u};  // bf16 -160
        const bf16x8 m160lo = __builtin_bit_cast(bf16x8, lo_half ? m160 : zero);
        const bf16x8 m160hi = __builtin_bit_cast(bf16x8, lo_half ? zero : m160);
        bf16x8 Blo[2], Bhi[2];
        float dlo[2], dhi[2];
        auto widen6 = [&](int i) {
            const uint32_t l0 = __builtin_amdgcn_alignbyte(o.l6[i][1], o.l6[i][0], m);
            const uint32_t l1 = __builtin_amdgcn_alignbyte(o.l6[i][2], o.l6[i][1], m);
            const uint32_t h0 = __builtin_amdgcn_alignbyte(o.h6[i][1], o.h6[i][0], m);
            const uint32_t h1 = __builtin_amdgcn_alignbyte(o.h6[i][2], o.h6[i][1], m);
            const uint32_t q0 = ((l0 >> nib) & 0x0F0F0F0Fu) | (((h0 >> hsh) & 0x03030303u) << 4);
            const uint32_t q1 = ((l1 >> nib) & 0x0F0F0F0Fu) | (((h1 >> hsh) & 0x03030303u) << 4);
            uint32_t cc[4];
            q4x4_bf16_128(q0, cc[0], cc[1]);
            q4x4_bf16_128(q1, cc[2], cc[3]);
            const u32x4 v = {cc[0], cc[1], cc[2], cc[3]};
            Blo[i] = __builtin_bit_cast(bf16x8, lo_half ? v : zero);
            Bhi[i] = __builtin_bit_cast(bf16x8, lo_half ? zero : v);
            // the row's scales of groups 2 kg, 2 kg + 1 of the chunk, and d
            const uint64_t sw = (((uint64_t)o.s6[i][1] << 32) | o.s6[i][0]) >> (8 * (m + 2 * kg));
            const float d = half_bits_to_float_fast(o.d6[i] >> (8 * m));
            dlo[i] = d * (float)(int)(int8_t)(sw & 0xFFu);
            dhi[i] = d * (float)(int)(int8_t)((sw >> 8) & 0xFFu);
        };
        f32x4 plo[3], phi[3];
        // MFMA pair k = 0 .. 2 MT - 1 is (row tile k / 2, column tile k % 2):
        // the -160 sum(x) starts depend on the row tile only, so the two
        // column tiles of a row tile take the same ones (six MFMAs per row
        // tile); both column tiles are widened before the first MFMA.
        auto fmas6 = [&](int k) {
            const int mt = k >> 1, nt = k & 1;
#pragma unroll
            for (int r = 0; r < 4; r++) {
                acc[mt][nt][r] = fmaf(dlo[nt], plo[k % 3][r], acc[mt][nt][r]);
                acc[mt][nt][r] = fmaf(dhi[nt], phi[k % 3][r], acc[mt][nt][r]);
            }
        };
        widen6(0);
        widen6(1);
        f32x4 tlo, thi;
#pragma unroll
        for (int k = 0; k < 2 * MT + 2; k++) {
            __builtin_amdgcn_sched_barrier(0);
            if (k < 2 * MT) {
                const int mt = k >> 1, nt = k & 1;
                const bf16x8 A = __builtin_bit_cast(bf16x8, o.a[mt]);
                if (nt == 0) {
                    ops_wait_row<MT>(mt, o);
                    tlo = mfma_bf16(A, m160lo);
                    thi = mfma_bf16(A, m160hi);
                }
                plo[k % 3] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, Blo[nt], tlo, 0, 0, 0);
                phi[k % 3] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(A, Bhi[nt], thi, 0, 0, 0);
            }
            if (k >= 2) fmas6(k - 2);
        }
    };

    // ---- pipeline ----------------------------------------------------------
    // Stage s sits in ring slot s % NS.  Iteration s: the loader waves wait
    // until their loads of stage s have landed (the later stages in flight
    // are those already issued), everyone meets at the barrier (stage s is in
    // LDS and the compute of s - 1 is done), then the loaders load stage
    // s + NS - 1 into slot (s - 1) % NS while the compute waves contract
    // stage s.  The compute waves issue no global loads, so they never wait
    // for room in the CU's queue of outstanding loads.  Nothing is loaded
    // past the split's last stage.
    if (wave >= 8) {
        for (int i = 0; i < NS - 1; i++)
            if (i < nst) issue(i);
        for (int s = 0; s < nst; s++) {
            // stages issued after s: min(nst - 1, s + NS - 2) - s
            const int later = nst - 1 - s < NS - 2 ? nst - 1 - s : NS - 2;
            loader_barrier_n<G::kLoads, NS - 2>(later);
            if (s + NS - 1 < nst) issue(s + NS - 1);
        }
    } else {
        for (int s = 0; s < nst; s++) {
            compute_barrier();
            if constexpr (T == kQ6_K)
                compute6(s);
            else
                compute(s);
        }
    }

    // ---- epilogue ----------------------------------------------------------
    // Block 1's waves hand their tiles to block 0's waves through the ring
    // (wave nq's quarter at 2 MT KiB nq); those add them (first-block sum +
    // second-block sum) and write the tile row-major into the ring (row pitch
    // kStagePitch floats); then the compute waves store whole rows, 16 bytes
    // a lane.  Every wave (the loaders too) passes the same barriers.
    __syncthreads();
    f32x4 *const hand = reinterpret_cast<f32x4 *>(ring + 2048 * MT * nq);
    if (wave < 8 && kg == 1) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++) hand[(mt * 2 + nt) * 64 + lane] = acc[mt][nt];
    }
    __syncthreads();
    if (wave < 8 && kg == 0) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++) acc[mt][nt] += hand[(mt * 2 + nt) * 64 + lane];
    }
    __syncthreads();
    float *const stage = reinterpret_cast<float *>(ring);
    if (wave < 8 && kg == 0) {
        // D layout of a 16 x 16 tile: lane holds column lane & 15, rows 4 (lane >> 4) + r.
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nt = 0; nt < 2; nt++)
#pragma unroll
                for (int r = 0; r < 4; r++)
                    stage[(16 * mt + 4 * lk + r) * kStagePitch + 32 * nq + 16 * nt + lr] = acc[mt][nt][r];
    }
    __syncthreads();
    // Split 0 writes Y, split k > 0 workspace partial k - 1 for the
    // reduction kernel.
    float *const out = split == 0 ? Y : part + (int64_t)(split - 1) * M * N;
    const int col = 4 * (tid & 31);
    if (tid >= kCompute) return;
#pragma unroll
    for (int pass = 0; pass < kTileM * 32 / kCompute; pass++) {
        const int row = 16 * pass + (tid >> 5);
        const int m = m0 + row, n = n0 + col;
        if (m >= M || n >= N) continue;
        const float4 val = *reinterpret_cast<const float4 *>(stage + row * kStagePitch + col);
        float *const dst = out + (int64_t)m * N + n;
        if ((N & 3) == 0) {
            // nontemporal: the tile is not read again by this kernel
            __builtin_nontemporal_store(f32x4{val.x, val.y, val.z, val.w}, reinterpret_cast<f32x4 *>(dst));
        } else {
            const float v4[4] = {val.x, val.y, val.z, val.w};
            for (int i = 0; i < 4 && n + i < N; i++) dst[i] = v4[i];
        }
    }
}

// y += part[0] + part[1] + ... + part[S - 2], in that order (4 floats a
// thread): every partial is loaded before the first add.
__global__ __launch_bounds__(256) void gemm_tile_reduce_kernel(const float *__restrict__ part, int S1,
                                                               int64_t mn, float *__restrict__ y) {
    const int64_t i = 4 * ((int64_t)blockIdx.x * blockDim.x + threadIdx.x);
    if (i >= mn) return;
    float4 b[7];
#pragma unroll
    for (int k = 0; k < 7; k++)
        if (k < S1) b[k] = *reinterpret_cast<const float4 *>(part + (int64_t)k * mn + i);
    float4 a = *reinterpret_cast<const float4 *>(y + i);
#pragma unroll
    for (int k = 0; k < 7; k++) {
        if (k < S1) {
            a.x += b[k].x;
            a.y += b[k].y;
            a.z += b[k].z;
            a.w += b[k].w;
        }
    }
    *reinterpret_cast<float4 *>(y + i) = a;
}

namespace {

// Row tiles of X per workgroup: the smallest of 1, 2, 4, 8 that covers M, so
// that small M computes no padding rows.  Q8_0 up to M = 128 with so few
// column tiles that 128-row tiles would split K eight ways takes 64-row
// tiles split four ways instead: three partial tiles per output in place of
// seven (M = 128, N = 4096: 18.7 against 19.7 us; the K-quant and Q4_0
// tiles at N = 14336 measured slower with 64 rows).
int tile_mt(int type_id, int M, int N) {
    if (M <= 16) return 1;
    if (M <= 32) return 2;
    if (M <= 64) return 4;
    if (type_id == kQ8_0 && M <= 128 && (N + kTileN - 1) / kTileN * 8 <= device_cus()) return 4;
    return 8;
}

int tile_splits(int type_id, int M, int N, int K, size_t workspace_bytes) {
    const int tm = 16 * tile_mt(type_id, M, N);
    const int tiles = (M + tm - 1) / tm * ((N + kTileN - 1) / kTileN);
    const int nst = K / 64;
    // A split holds a whole number of four-stage rounds (and so of Q4_K
    // superblocks).
    int S = 1;
    while (S < 8 && tiles * 2 * S <= device_cus() && nst % (8 * S) == 0 &&
           (size_t)(2 * S - 1) * M * N * sizeof(float) <= workspace_bytes)
        S *= 2;
    return S;
}

}  // namespace

bool gemm_tile_supported(int type_id, int64_t row_bytes, int M, int N, int K, const void *w,
                         const void *x, const void *y) {
    if (type_id != kQ8_0 && type_id != kQ4_0 && type_id != kQ4_K && type_id != kQ5_K && type_id != kQ6_K)
        return false;
    if (M <= 0 || N <= 0 || K % 256 != 0) return false;
    if (((reinterpret_cast<uintptr_t>(w) | (uintptr_t)row_bytes) & 3u) != 0) return false;
    if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0 || (reinterpret_cast<uintptr_t>(y) & 15u) != 0) return false;
    // 32-bit buffer offsets: a tile's rows of X and W
    return (int64_t)kTileMMax * K * 2 < ((int64_t)1 << 31) && (int64_t)kTileN * row_bytes < ((int64_t)1 << 31);
}

size_t gemm_tile_workspace_bytes(int type_id, int M, int N, int K) {
    const int S = tile_splits(type_id, M, N, K, (size_t)-1);
    return S > 1 ? (size_t)(S - 1) * M * N * sizeof(float) : 0;
}

hipError_t launch_gemm_tile(int type_id, const uint8_t *w, int64_t row_bytes, const uint16_t *x,
                            float *y, int M, int N, int K, hipStream_t stream, float *workspace,
                            size_t workspace_bytes) {
    if (M <= 0) return hipSuccess;
    int S = tile_splits(type_id, M, N, K, workspace != nullptr ? workspace_bytes : 0);
    if (((int64_t)M * N) % 4 != 0 || (reinterpret_cast<uintptr_t>(workspace) & 15u) != 0) S = 1;
    const int mt = tile_mt(type_id, M, N), tm = 16 * mt;
    const unsigned tiles = (unsigned)(((M + tm - 1) / tm) * ((N + kTileN - 1) / kTileN));
    const dim3 grid(tiles * (unsigned)S), block(kThreads);
    float *part = S > 1 ? workspace : nullptr;
#define GOLLEK_TILE_LAUNCH(TY)                                                                        \
    do {                                                                                              \
        if (mt == 1)                                                                                  \
            hipLaunchKernelGGL((gemm_tile_kernel<TY, 1>), grid, block, 0, stream, w, row_bytes, x, y, M, N, \
                               K, S, part);                                                           \
        else if (mt == 2)                                                                             \
            hipLaunchKernelGGL((gemm_tile_kernel<TY, 2>), grid, block, 0, stream, w, row_bytes, x, y, M, N, \
                               K, S, part);                                                           \
        else if (mt == 4)                                                                             \
            hipLaunchKernelGGL((gemm_tile_kernel<TY, 4>), grid, block, 0, stream, w, row_bytes, x, y, M, N, \
                               K, S, part);                                                           \
        else                                                                                          \
            hipLaunchKernelGGL((gemm_tile_kernel<TY, 8>), grid, block, 0, stream, w, row_bytes, x, y, M, N, \
                               K, S, part);                                                           \
    } while (0)
    switch (type_id) {
    case kQ8_0:
        GOLLEK_TILE_LAUNCH(kQ8_0);
        break;
    case kQ4_0:
        GOLLEK_TILE_LAUNCH(kQ4_0);
        break;
    case kQ4_K:
        GOLLEK_TILE_LAUNCH(kQ4_K);
        break;
    case kQ5_K:
        GOLLEK_TILE_LAUNCH(kQ5_K);
        break;
    case kQ6_K:
        GOLLEK_TILE_LAUNCH(kQ6_K);
        break;
    default:
        return hipErrorInvalidValue;
    }
#undef GOLLEK_TILE_LAUNCH
    if (S > 1) {
        const int64_t mn = (int64_t)M * N;
        hipLaunchKernelGGL(gemm_tile_reduce_kernel, dim3((unsigned)((mn / 4 + 255) / 256)), dim3(256), 0,
                           stream, part, S - 1, mn, y);
    }
    return hipGetLastError();
}

}  // namespace gollek
