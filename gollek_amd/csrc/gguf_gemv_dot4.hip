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
// Layout: 4 lanes cover one 144-byte superblock; lane g of the four uses
// the header and the 32 quant bytes of chunk g (elements 64g..64g+31 in the
// low nibbles, 64g+32..64g+63 in the high nibbles), so a lane always works
// on the same 64 columns and keeps their x digits in registers.  One row per
// wave pass (up to 16 superblocks = 64 lanes).
//
// Streaming: each wave owns a ring of kRingSlots rows in LDS.  Rows arrive by
// buffer->LDS loads of whole kilobytes (contiguous, nontemporal, no
// registers held while in flight); a wave waits for the oldest row, reads its
// lane's 48 bytes, refills the slot with the row kRingSlots ahead and only
// then computes, so the loads of later rows overlap the arithmetic.  The
// x loads are issued before the first ring loads, and the workgroup turns x
// into digit planes while the rows stream in.  Row results collect in one
// register (lane i holds the wave's row i) and are stored once at the end:
// stores in the loop would share the load counter the ring waits on.
#include "gguf_dot4.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

namespace {

constexpr int kRingWaves = 8;      // waves per workgroup (one workgroup per CU)
constexpr int kRingSlots = 4;      // rows in flight per wave
constexpr int kMaxWaveRows = 64;   // rows per wave (one result register)
constexpr int kMaxGroups = 16 * 8; // 32-element groups of x (K <= 4096)

}  // namespace

// NDMA = kilobytes per row slot (row_bytes <= 1024 * NDMA).
template <int NDMA>
__global__ __launch_bounds__(kRingWaves * 64) void gemv_q4_k_dot4_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes64, int nsb, const float *__restrict__ x,
    float *__restrict__ y, int64_t rows) {
    constexpr int kSlot = 1024 * NDMA;
    constexpr int kThreads = kRingWaves * 64;
    constexpr int XL = (8 * kMaxGroups + kThreads - 1) / kThreads;
    __shared__ __attribute__((aligned(16))) uint32_t digs[(kDigitWords + 2) * kMaxGroups];
    __shared__ __attribute__((aligned(16))) uint8_t ring[kRingWaves * kRingSlots * kSlot];

    const int ngroups = nsb * 8;
    uint32_t *dig = digs;
    float *scl = reinterpret_cast<float *>(digs + kDigitWords * ngroups);
    float *gsum = scl + ngroups;
    const uint32_t row_bytes = (uint32_t)row_bytes64;
    const int lane = threadIdx.x & 63;
    const int wib = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int64_t nwaves = (int64_t)gridDim.x * kRingWaves;
    const int64_t wave = (int64_t)blockIdx.x * kRingWaves + wib;
    const int64_t row_base = wave_uniform(wave * rows / nwaves);
    const int64_t row_end = wave_uniform((wave + 1) * rows / nwaves);
    const int nrows = (int)(row_end - row_base);  // <= kMaxWaveRows (host grid choice)
    // The host keeps (row_end - row_base) * row_bytes < 2^31.
    const __amdgpu_buffer_rsrc_t rs = wave_buffer(w + row_base * row_bytes64, (uint32_t)nrows * row_bytes);
    uint8_t *myring = ring + wib * (kRingSlots * kSlot);

    XPart<XL> xp;
    load_x_parts<kThreads, XL>(xp, x, ngroups);
    __builtin_amdgcn_sched_barrier(0);  // every x load ahead of the ring loads
#pragma unroll
    for (int j = 0; j < kRingSlots; j++)
        row_to_lds<NDMA>(rs, myring + j * kSlot, j < nrows ? (uint32_t)j * row_bytes : kMaskedOffset,
                         row_bytes, lane);
    store_x_digits<kThreads, XL>(xp, ngroups, dig, scl, gsum);
    // LDS-only exchange: wait for this wave's digit stores, then the barrier
    // (no wait on the ring loads, which are still in flight).
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();

    const int g = lane & 3;
    const int sb = lane >> 2;
    const bool act = sb < nsb;
    uint32_t dg[2][3][8];
    float sg[2], xg[2];
    load_lane_digits(dig, scl, gsum, sb, g, act, dg, sg, xg);

    // Lanes past the row's superblocks read superblock 0 and are masked.
    const uint32_t a_h = (uint32_t)(uintptr_t)(lds_ptr)myring + (act ? sb : 0) * kQKBlockBytes;
    const uint32_t a_q = a_h + 16 + 32 * g;
    float res = 0.0f;
    for (int r0 = 0; r0 < nrows; r0 += kRingSlots) {
#pragma unroll
        for (int j = 0; j < kRingSlots; j++) {
            u32x4 hd, qa, qb;
            // Reads of the ring go through inline asm: the compiler cannot tell
            // which buffer->LDS load wrote which bytes and would wait for all
            // of them.  Row r0 + j is complete once the (kRingSlots - 1) rows
            // issued after it are the only loads outstanding; the block waits
            // for its own LDS reads before the slot is refilled.
            asm volatile("s_waitcnt vmcnt(%6)\n\t"
                         "ds_read_b128 %0, %3 offset:%7\n\t"
                         "ds_read_b128 %1, %4 offset:%7\n\t"
                         "ds_read_b128 %2, %5 offset:%7\n\t"
                         "s_waitcnt lgkmcnt(0)"
                         : "=&v"(hd), "=&v"(qa), "=&v"(qb)
                         : "v"(a_h), "v"(a_q), "v"(a_q + 16), "n"(NDMA * (kRingSlots - 1)),
                           "n"(j * kSlot)
                         : "memory");
            const int next = r0 + j + kRingSlots;
            row_to_lds<NDMA>(rs, myring + j * kSlot,
                             next < nrows ? (uint32_t)next * row_bytes : kMaskedOffset, row_bytes,
                             lane);
            float acc = q4k_dot4_row(to_uint4(hd), to_uint4(qa), to_uint4(qb), dg, sg, xg, g);
            acc = wave_sum_to_lane63(act ? acc : 0.0f);
            const float tot =
                __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, acc), 63));
            res = lane == r0 + j ? tot : res;
        }
    }
    // Drain the (masked) ring loads before the workgroup's LDS is released.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    if (lane < nrows) y[row_base + lane] = res;
}

namespace {

template <int NDMA>
hipError_t launch_ring(const uint8_t *w, int64_t row_bytes, int nsb, const float *x, float *y,
                       int64_t rows, hipStream_t stream) {
    const int64_t cus = device_cus();
    // One workgroup per CU when that keeps every wave at <= kMaxWaveRows rows;
    // fewer when there are fewer rows than waves; more (run in turn) for
    // very tall matrices.
    int64_t grid = (rows + kRingWaves - 1) / kRingWaves;
    if (grid > cus) grid = cus;
    const int64_t per_wave_max = kRingWaves * (int64_t)kMaxWaveRows;
    if (grid * per_wave_max < rows) grid = (rows + per_wave_max - 1) / per_wave_max;
    hipLaunchKernelGGL((gemv_q4_k_dot4_kernel<NDMA>), dim3((unsigned)grid), dim3(kRingWaves * 64), 0,
                       stream, w, row_bytes, nsb, x, y, rows);
    return hipGetLastError();
}

}  // namespace

bool q4k_dot4_supported(int64_t row_bytes, int64_t cols, int64_t rows, const void *w,
                        const float *x) {
    (void)rows;  // a wave's descriptor spans <= 64 rows of <= 2304 bytes
    if (tuning().gemv_variant == 1) return false;  // forced fp32 path
    const int64_t nsb = cols / kQK;
    return nsb >= 1 && nsb <= 16 && row_bytes == nsb * kQKBlockBytes &&
           (reinterpret_cast<uintptr_t>(w) & 15u) == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

hipError_t launch_gemv_q4k_dot4(const uint8_t *w, int64_t row_bytes, int64_t cols,
                                const float *x, float *y, int64_t rows, hipStream_t stream) {
    const int nsb = (int)(cols / kQK);
    if (row_bytes <= 1024) return launch_ring<1>(w, row_bytes, nsb, x, y, rows, stream);
    if (row_bytes <= 2048) return launch_ring<2>(w, row_bytes, nsb, x, y, rows, stream);
    return launch_ring<3>(w, row_bytes, nsb, x, y, rows, stream);
}

}  // namespace gollek
