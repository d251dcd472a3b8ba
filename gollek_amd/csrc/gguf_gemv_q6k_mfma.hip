// gguf_gemv_q6k_mfma.hip -- Q6_K GEMV (decode, M = 1) on the gfx950 matrix
// cores, K a multiple of 2048 up to 14336 (Q4_K_M files store the lm_head
// and part of the FFN down projections as Q6_K).
//
// Same value as the reference raw Q6_K mat-vec (RT/GgufQ6RawDot.java:32-134;
// block layout RT/GgufKBlockDequantizer.java:319-432): per 256-element
// superblock, ql[128] low nibbles, qh[64] two high bits, scales[16] (int8,
// one per 16 elements) and an fp16 d;
//   y[n] = sum_sb d sum_j sc_j sum_{i in j} (q_i - 32) x_i.
// Tolerance parity (rel_err <= 1e-3 against the fp64 dot, as the other
// GEMVs).
//
// Contraction.  v_mfma_i32_16x16x64_i8 of 16 weight rows (B: 6-bit codes
// 0..63 as bytes) against 64 columns of x held as four balanced signed-byte
// digit planes of 30-bit integers (the Q4_K kernels' x, x_planes4).  Chunk c
// of a superblock (half ip = c >> 1, part = c & 1) covers elements
// 128 ip + 32 part + l and + 64 (l < 32): B lane n + 16 g holds, for
// l = 8 g .. 8 g + 7, the codes of the first run in bytes 0..7 (ql's low
// nibble and qh bits 2 part, 2 part + 1) and of the second in bytes 8..15
// (ql's high nibble, qh bits 4 + 2 part, 5 + 2 part).  The 16-element
// scales need one output per 16 columns, so A row m = 4 q + p holds plane
// p of quarter q (run q >> 1, l in 16 (q & 1) .. + 15), live on the lanes g
// with g >> 1 == q & 1 and zero elsewhere; output lane n + 16 g then holds
// row n's four plane sums of quarter g, each exact in int32.  The -32
// offset is applied per plane in int32 before the planes are combined
// (D_p - 32 sum of the quarter's digits of plane p), so it adds no
// rounding; the planes combine as (D2 + 256 D3) 65536 + (D0 + 256 D1) in
// fp32, then scale by sc_q and, per superblock, by d and x's scale.
//
// Streaming.  One workgroup (16 waves) per CU takes an equal share of the
// rows in 16-row tiles.  An item is a tile's 16 rows x 8 superblocks (an
// eighth of a row per 2048 columns: 1680 bytes of each row, 26,880 bytes);
// every wave issues two of an item's 27 buffer->LDS loads of 1 KB, one
// barrier per item publishes it, and wave w works on position w & 7 of the
// items j with j & 1 == w >> 3.  K <= 4096: wave w owns superblock w, builds
// its x operands once, and a 5-slot ring keeps four items (107 KB) in
// flight per CU.  Wider K: x's digit planes for every superblock are built
// once into LDS (1 KB each), a wave reads its operands per item, and the
// ring has 3 slots (carrying x in the items instead, converted per item,
// with a 4-slot ring measured 19.8 us against 17.4 us at 4096 x 14336: the
// conversion sits on every item's critical path).  A wave sums its items
// of a tile in registers; the waves' row sums meet in LDS and one wave per
// tile adds them.  Superblocks are
// 210 bytes, so every other one starts 2 bytes off a dword in LDS: a lane
// reads aligned dwords and v_alignbyte_b32 realigns them (the shift is 0 or
// 2, uniform per wave).
#include "gguf_mfma_q4k.hpp"

namespace gollek {

using namespace mfq;

namespace {

constexpr int kQ6TileRows = 16;  // rows per MFMA tile
constexpr int kQ6Waves = 16;
constexpr int kQ6Threads = kQ6Waves * 64;
constexpr int kQ6SbBytes = 210;
constexpr int kQ6HalfSb = 8;                                     // superblocks per item
constexpr int kQ6Pitch = kQ6HalfSb * kQ6SbBytes;                 // 1680: 105 16-byte units (odd)
constexpr int kQ6Item = kQ6TileRows * kQ6Pitch;                    // 26880
constexpr int kQ6Dma = (kQ6Item + 1023) / 1024;                  // 27 loads of 1 KB
constexpr int kQ6DmaPerWave = (kQ6Dma + kQ6Waves - 1) / kQ6Waves;  // 2
constexpr int kQ6Slot = kQ6Dma * 1024;
constexpr int kQ6MaxRows = 1024;                                 // rows per workgroup
constexpr int kQ6MaxSbLds = 56;                                  // superblocks of x in LDS (K <= 14336)

// One superblock's x operands from its four digit planes (1 KB of LDS,
// plane p at + 256 p, element i at byte i).  A lane (m, g): plane p = m & 3
// of quarter q = m >> 2 of chunk c, i.e. elements 128 (c >> 1) + 32 (c & 1)
// + 64 (q >> 1) + 8 g .. + 7, live when g >> 1 == q & 1 (bytes 0..7 for
// q < 2, 8..15 otherwise); corr[c][p] = 32 x the digit sum of plane p over
// this output lane's quarter g of chunk c.
__device__ __forceinline__ void q6_x_operands(uint32_t planes, i32x4 (&A)[4], int (&corr)[4][4]) {
    const int lane = threadIdx.x & 63;
    const int n = lane & 15, g = lane >> 4, q = n >> 2, pl = n & 3;
    const bool live = (g >> 1) == (q & 1);
    uint2 xa[4];
    uint4 qs[4][4];  // [c][p]: the 16 digits of this lane's quarter
    const uint32_t a_x = planes + 256u * pl + 64u * (q >> 1) + 8u * g;
    const uint32_t a_s = planes + 64u * (g >> 1) + 16u * (g & 1);
    asm volatile(
        "s_waitcnt lgkmcnt(0)\n\t"
        "ds_read_b64 %0, %20\n\t"
        "ds_read_b64 %1, %20 offset:32\n\t"
        "ds_read_b64 %2, %20 offset:128\n\t"
        "ds_read_b64 %3, %20 offset:160\n\t"
        "ds_read_b128 %4, %21\n\t"
        "ds_read_b128 %5, %21 offset:256\n\t"
        "ds_read_b128 %6, %21 offset:512\n\t"
        "ds_read_b128 %7, %21 offset:768\n\t"
        "ds_read_b128 %8, %21 offset:32\n\t"
        "ds_read_b128 %9, %21 offset:288\n\t"
        "ds_read_b128 %10, %21 offset:544\n\t"
        "ds_read_b128 %11, %21 offset:800\n\t"
        "ds_read_b128 %12, %21 offset:128\n\t"
        "ds_read_b128 %13, %21 offset:384\n\t"
        "ds_read_b128 %14, %21 offset:640\n\t"
        "ds_read_b128 %15, %21 offset:896\n\t"
        "ds_read_b128 %16, %21 offset:160\n\t"
        "ds_read_b128 %17, %21 offset:416\n\t"
        "ds_read_b128 %18, %21 offset:672\n\t"
        "ds_read_b128 %19, %21 offset:928\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(xa[0]), "=&v"(xa[1]), "=&v"(xa[2]), "=&v"(xa[3]), "=&v"(qs[0][0]), "=&v"(qs[0][1]),
          "=&v"(qs[0][2]), "=&v"(qs[0][3]), "=&v"(qs[1][0]), "=&v"(qs[1][1]), "=&v"(qs[1][2]),
          "=&v"(qs[1][3]), "=&v"(qs[2][0]), "=&v"(qs[2][1]), "=&v"(qs[2][2]), "=&v"(qs[2][3]),
          "=&v"(qs[3][0]), "=&v"(qs[3][1]), "=&v"(qs[3][2]), "=&v"(qs[3][3])
        : "v"(a_x), "v"(a_s)
        : "memory");
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int lo = live ? (int)xa[c].x : 0, hi = live ? (int)xa[c].y : 0;
        A[c] = q < 2 ? i32x4{lo, hi, 0, 0} : i32x4{0, 0, lo, hi};
#pragma unroll
        for (int p = 0; p < 4; p++) {
            const uint4 d = qs[c][p];
            int sum = __builtin_amdgcn_sdot4((int)d.x, 0x01010101, 0, false);
            sum = __builtin_amdgcn_sdot4((int)d.y, 0x01010101, sum, false);
            sum = __builtin_amdgcn_sdot4((int)d.z, 0x01010101, sum, false);
            sum = __builtin_amdgcn_sdot4((int)d.w, 0x01010101, sum, false);
            corr[c][p] = 32 * sum;
        }
    }
}

// K > 4096: the -32 corrections of one superblock, for q6_x_operands_sums.
// wd[p] = this lane's four digits of plane p (x_planes4; lane l holds
// elements 4 l .. 4 l + 3), so group G = l >> 2 of 16 elements is a quad:
// quarter g of chunk c with G = 8 (c >> 1) + 2 (c & 1) + 4 (g >> 1) + (g &
// 1).  With s_p its digit sum of plane p (|s_p| <= 16 x 128), the pair
// {32 (s0 + 256 s1), 32 (s2 + 256 s3)} (|.| < 2^24) goes to sums + 8 (4 g
// + c): what the plane pairs (D0 + 256 D1, D2 + 256 D3) of a chunk lose to
// the -32 offset.
__device__ __forceinline__ void q6_digit_sums(const uint32_t (&wd)[4], uint32_t sums) {
    const int lane = threadIdx.x & 63;
    int gs[4];
#pragma unroll
    for (int p = 0; p < 4; p++) {
        int t = __builtin_amdgcn_sdot4((int)wd[p], 0x01010101, 0, false);
        t += dpp_i<0xB1>(t);  // quad_perm [1,0,3,2]
        t += dpp_i<0x4E>(t);  // quad_perm [2,3,0,1]
        gs[p] = t;
    }
    const int G = lane >> 2;
    const int c = 2 * (G >> 3) + ((G >> 1) & 1), g = 2 * ((G >> 2) & 1) + (G & 1);
    const uint32_t lo = (uint32_t)(32 * (gs[0] + 256 * gs[1]));
    const uint32_t hi = (uint32_t)(32 * (gs[2] + 256 * gs[3]));
    if ((lane & 3) == 0)
        asm volatile("ds_write_b64 %0, %1" : : "v"(sums + 8u * (uint32_t)(4 * g + c)), "v"(uint2{lo, hi}) : "memory");
}

// K > 4096: one superblock's operands from its planes and q6_digit_sums'
// table.  a01 / a23: this lane's A bytes in the planes (plane base +
// 256 p + 64 (q >> 1) + 8 g) for the lanes whose A row is live in dwords
// 0, 1 (q < 2) / 2, 3 (q >= 2), a zeroed block otherwise, so the halves of A
// need no selects; cc[c] = the chunk's two corrections for quarter g.
__device__ __forceinline__ void q6_x_operands_sums(uint32_t a01, uint32_t a23, uint32_t sums, i32x4 (&A)[4],
                                                   int (&cc)[4][2]) {
    const int g = (threadIdx.x & 63) >> 4;
    uint2 x01[4], x23[4];
    uint4 sv[2];
    asm volatile(
        "s_waitcnt lgkmcnt(0)\n\t"
        "ds_read_b64 %0, %10\n\t"
        "ds_read_b64 %1, %10 offset:32\n\t"
        "ds_read_b64 %2, %10 offset:128\n\t"
        "ds_read_b64 %3, %10 offset:160\n\t"
        "ds_read_b64 %4, %11\n\t"
        "ds_read_b64 %5, %11 offset:32\n\t"
        "ds_read_b64 %6, %11 offset:128\n\t"
        "ds_read_b64 %7, %11 offset:160\n\t"
        "ds_read_b128 %8, %12\n\t"
        "ds_read_b128 %9, %12 offset:16\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(x01[0]), "=&v"(x01[1]), "=&v"(x01[2]), "=&v"(x01[3]), "=&v"(x23[0]), "=&v"(x23[1]),
          "=&v"(x23[2]), "=&v"(x23[3]), "=&v"(sv[0]), "=&v"(sv[1])
        : "v"(a01), "v"(a23), "v"(sums + 32u * g)
        : "memory");
#pragma unroll
    for (int c = 0; c < 4; c++) A[c] = i32x4{(int)x01[c].x, (int)x01[c].y, (int)x23[c].x, (int)x23[c].y};
    cc[0][0] = (int)sv[0].x;
    cc[0][1] = (int)sv[0].y;
    cc[1][0] = (int)sv[0].z;
    cc[1][1] = (int)sv[0].w;
    cc[2][0] = (int)sv[1].x;
    cc[2][1] = (int)sv[1].y;
    cc[3][0] = (int)sv[1].z;
    cc[3][1] = (int)sv[1].w;
}

}  // namespace

// XLDS: K > 4096, x's planes and digit sums for every superblock in LDS.
template <bool XLDS>
__global__ __launch_bounds__(kQ6Threads) void gemv_q6_k_mfma_tile_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes64, int nsb, const float *__restrict__ x,
    float *__restrict__ y, int64_t rows, int64_t rows_per_wg) {
    constexpr int kQ6Slots = XLDS ? 3 : 5;
    static_assert(kQ6DmaPerWave * kQ6Waves >= kQ6Dma, "item loads");
    static_assert(kQ6Waves * 1024 <= kQ6Slot, "x scratch fits a slot");
    __shared__ __attribute__((aligned(16))) uint8_t ring[kQ6Slots * kQ6Slot + 1024];  // + sink
    __shared__ float part[2][kQ6Waves][2][16];  // [tile & 1][wave][quarter pair][row]
    __shared__ float yout[kQ6MaxRows];
    __shared__ __attribute__((aligned(16))) uint8_t xpl[XLDS ? kQ6MaxSbLds : 1][1024];  // XLDS: x's planes
    __shared__ float xst[XLDS ? kQ6MaxSbLds : 1];                                      // XLDS: x's scales
    __shared__ __attribute__((aligned(16))) int32_t xds[XLDS ? kQ6MaxSbLds : 1][32];   // XLDS: corrections
    __shared__ __attribute__((aligned(16))) uint32_t zpad[XLDS ? 64 : 1];              // XLDS: zeros for A
    // K <= 4096: each wave's x scratch (four digit planes, 1 KB) is kilobyte
    // w of the last ring slot, which the loop first refills after every wave
    // has read its operands back.
    const uint32_t xscr = (uint32_t)(uintptr_t)(lds_ptr)(ring + (kQ6Slots - 1) * kQ6Slot);

    const uint32_t row_bytes = (uint32_t)row_bytes64;
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_wg;
    const int nr = (int)(rows - r0 < rows_per_wg ? rows - r0 : rows_per_wg);  // 1..kQ6MaxRows
    const int tiles = (nr + kQ6TileRows - 1) / kQ6TileRows;
    const int chunks = nsb / kQ6HalfSb;  // items per tile
    const int items = tiles * chunks;
    // Rows past the workgroup's share are out of the descriptor's range.
    const __amdgpu_buffer_rsrc_t rs = wave_buffer(w + r0 * row_bytes64, (uint32_t)nr * row_bytes);

    // This wave's item loads: load k = wv + 16 i moves staged bytes 1024 k + 16 lane
    // (row b / pitch, column b % pitch of the item's half); loads past the item
    // write the sink.
    uint32_t dbase[kQ6DmaPerWave];
#pragma unroll
    for (int i = 0; i < kQ6DmaPerWave; i++) {
        const uint32_t k = (uint32_t)(wv + kQ6Waves * i);
        const uint32_t b = 1024u * k + 16u * lane;
        const uint32_t r = b / kQ6Pitch, col = b - r * kQ6Pitch;
        dbase[i] = (k < (uint32_t)kQ6Dma && r < (uint32_t)kQ6TileRows) ? r * row_bytes + col : kMaskedOffset;
    }
    auto issue = [&](int slot, int item) {
        const int t = item / chunks, hf = item - t * chunks;
        const uint32_t uoff =
            item < items ? (uint32_t)t * kQ6TileRows * row_bytes + (uint32_t)hf * kQ6Pitch : kMaskedOffset;
#pragma unroll
        for (int i = 0; i < kQ6DmaPerWave; i++) {
            const int k = wv + kQ6Waves * i;
            uint8_t *dst = k < kQ6Dma ? ring + slot * kQ6Slot + 1024 * k : ring + kQ6Slots * kQ6Slot;
            const uint32_t o = (dbase[i] != kMaskedOffset && uoff != kMaskedOffset) ? dbase[i] + uoff : kMaskedOffset;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)dst, 16, o, 0, 0, kStreamLoad);
        }
    };

    const int sb = wv;
    const bool active = XLDS || sb < nsb;  // wave-uniform
    const int my_par = sb >> 3;
    float4 xr = {0.0f, 0.0f, 0.0f, 0.0f};
    constexpr int kXl = (kQ6MaxSbLds + kQ6Waves - 1) / kQ6Waves;  // x superblocks per wave (XLDS)
    float4 xq[XLDS ? kXl : 1];
    if constexpr (!XLDS) {
        const float4 xv = reinterpret_cast<const float4 *>(x)[64 * (active ? sb : 0) + lane];
        __builtin_amdgcn_sched_barrier(0);
        issue(0, 0);
        xr = xv;  // the conversion stays below the first item's loads
        asm volatile("" : "+v"(xr.x), "+v"(xr.y), "+v"(xr.z), "+v"(xr.w));
    } else {
        // Every x superblock of the wave first (w, w + 16, ...; past nsb the
        // last one again, unused), then the ring's first items: one round
        // trip for all of them instead of one per superblock.
#pragma unroll
        for (int i = 0; i < kXl; i++) {
            const int s2 = wv + kQ6Waves * i;
            xq[i] = reinterpret_cast<const float4 *>(x)[64 * (s2 < nsb ? s2 : nsb - 1) + lane];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int j = 0; j < kQ6Slots - 1; j++) issue(j, j);
        __builtin_amdgcn_sched_barrier(0);
    }

    // K <= 4096: wave w owns superblock w (item parity w >> 3, position
    // w & 7 in the item); a wave past nsb converts superblock 0 (its
    // operands are never used).  Wider K: wave w converts superblocks
    // w, w + 16, ... into xpl.
    const int n = lane & 15, g = lane >> 4;
    i32x4 A[4];
    int cc[4][2];  // per chunk: the corrections of (D0 + 256 D1, D2 + 256 D3)
    float xs = 0.0f;
    if constexpr (!XLDS) {
        const float v[4] = {xr.x, xr.y, xr.z, xr.w};
        uint32_t wd[4];
        const uint32_t myscr = xscr + 1024u * (uint32_t)wv;
        xs = x_planes4(v, myscr, wd);
        int corr[4][4];
        q6_x_operands(myscr, A, corr);
#pragma unroll
        for (int c = 0; c < 4; c++) {
            cc[c][0] = corr[c][0] + 256 * corr[c][1];
            cc[c][1] = corr[c][2] + 256 * corr[c][3];
        }
    } else {
        if (wv == 0) zpad[lane] = 0u;  // published by the first item's barrier
#pragma unroll
        for (int i = 0; i < kXl; i++) {
            const int s2 = wv + kQ6Waves * i;
            if (s2 < nsb) {  // uniform
                const float v[4] = {xq[i].x, xq[i].y, xq[i].z, xq[i].w};
                uint32_t wd[4];
                const float sc = x_planes4(v, (uint32_t)(uintptr_t)(lds_ptr)xpl[s2], wd);
                if (lane == 0) xst[s2] = sc;
                q6_digit_sums(wd, (uint32_t)(uintptr_t)(lds_ptr)xds[s2]);
            }
        }
    }
    if constexpr (!XLDS) {
#pragma unroll
        for (int j = 1; j < kQ6Slots - 1; j++) issue(j, j);
    }

    float acc = 0.0f;  // this wave's sum over its items of the current tile
    const uint32_t ring_base = (uint32_t)(uintptr_t)(lds_ptr)ring;
    // This wave's superblock within a row of an item, and its dword misalignment.
    const uint32_t sb_off = (uint32_t)(sb & 7) * kQ6SbBytes;
    const uint32_t sh = sb_off & 3u;  // 0 or 2
    const uint32_t row_al = ring_base + (uint32_t)n * kQ6Pitch + (sb_off & ~3u);
    const int hs = g >> 1, hh = g & 1;  // output quarter: run hs, half hh
    // XLDS: this lane's A bytes within a superblock's planes, and which half
    // of A they fill (none for the lanes whose row is dead in its run)
    const int aq = n >> 2;
    const bool live_a = (g >> 1) == (aq & 1);
    const uint32_t a_off = 256u * (uint32_t)(n & 3) + 64u * (uint32_t)(aq >> 1) + 8u * (uint32_t)g;
    const uint32_t zaddr = (uint32_t)(uintptr_t)(lds_ptr)zpad;
    const i32x4 zero4 = {0, 0, 0, 0};
    int slot = 0;
    for (int it = 0; it < items; it++) {
        // This wave's loads of item it are done once the later items' loads
        // are the only ones outstanding; the barrier makes every wave's
        // visible and ends every wave's reads of the slot refilled below.
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kQ6DmaPerWave * (kQ6Slots - 2)) : "memory");
        const int t = it / chunks, hf = it - t * chunks;
        // the previous tile's rows, once every wave's share is in part[]
        if (hf == 0 && t >= 1 && wv == (t - 1) % kQ6Waves && lane < 16) {
            float s = 0.0f;
            for (int k = 0; k < min(nsb, kQ6Waves); k++)
                s += part[(t - 1) & 1][k][0][lane] + part[(t - 1) & 1][k][1][lane];
            const int row = (t - 1) * kQ6TileRows + lane;
            if (row < nr) yout[row] = s;
        }
        issue(slot == 0 ? kQ6Slots - 1 : slot - 1, it + kQ6Slots - 1);
        if (active && (hf & 1) == my_par) {
            if constexpr (XLDS) {
                const int s2 = kQ6HalfSb * hf + (sb & 7);
                const uint32_t pa = (uint32_t)(uintptr_t)(lds_ptr)xpl[s2] + a_off;
                q6_x_operands_sums(live_a && aq < 2 ? pa : zaddr, live_a && aq >= 2 ? pa : zaddr,
                                   (uint32_t)(uintptr_t)(lds_ptr)xds[s2], A, cc);
                xs = xst[s2];
            }
            const uint32_t ab = row_al + (uint32_t)slot * kQ6Slot;
            const uint32_t aq = ab + 8u * g;
            // ql pieces (c = 0..3 at 0, 32, 64, 96), qh pieces (ip = 0, 1 at
            // 128, 160), the 16 scale bytes at 192 and d at 208; three
            // dwords per 8-byte piece, realigned by sh bytes.
            uint2 p01[6], s01, s23;  // dwords 0, 1 of each piece; scale dwords
            uint32_t p2[6], s4;        // dword 2 of each piece; the dword holding d
            asm volatile(
                "ds_read2_b32 %0, %15 offset1:1\n\t"
                "ds_read_b32 %6, %15 offset:8\n\t"
                "ds_read2_b32 %1, %15 offset0:8 offset1:9\n\t"
                "ds_read_b32 %7, %15 offset:40\n\t"
                "ds_read2_b32 %2, %15 offset0:16 offset1:17\n\t"
                "ds_read_b32 %8, %15 offset:72\n\t"
                "ds_read2_b32 %3, %15 offset0:24 offset1:25\n\t"
                "ds_read_b32 %9, %15 offset:104\n\t"
                "ds_read2_b32 %4, %15 offset0:32 offset1:33\n\t"
                "ds_read_b32 %10, %15 offset:136\n\t"
                "ds_read2_b32 %5, %15 offset0:40 offset1:41\n\t"
                "ds_read_b32 %11, %15 offset:168\n\t"
                "ds_read2_b32 %12, %16 offset0:48 offset1:49\n\t"
                "ds_read2_b32 %13, %16 offset0:50 offset1:51\n\t"
                "ds_read_b32 %14, %16 offset:208\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(p01[0]), "=&v"(p01[1]), "=&v"(p01[2]), "=&v"(p01[3]), "=&v"(p01[4]), "=&v"(p01[5]),
                  "=&v"(p2[0]), "=&v"(p2[1]), "=&v"(p2[2]), "=&v"(p2[3]), "=&v"(p2[4]), "=&v"(p2[5]),
                  "=&v"(s01), "=&v"(s23), "=&v"(s4)
                : "v"(aq), "v"(ab)
                : "memory");
            uint32_t ql[4][2], qh[2][2];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                ql[c][0] = __builtin_amdgcn_alignbyte(p01[c].y, p01[c].x, sh);
                ql[c][1] = __builtin_amdgcn_alignbyte(p2[c], p01[c].y, sh);
            }
#pragma unroll
            for (int ip = 0; ip < 2; ip++) {
                qh[ip][0] = __builtin_amdgcn_alignbyte(p01[4 + ip].y, p01[4 + ip].x, sh);
                qh[ip][1] = __builtin_amdgcn_alignbyte(p2[4 + ip], p01[4 + ip].y, sh);
            }
            // scale bytes 0..15 (s0..s3, realigned) and d (2 bytes at byte sh of s4)
            const uint32_t s0 = __builtin_amdgcn_alignbyte(s01.y, s01.x, sh);
            const uint32_t s1 = __builtin_amdgcn_alignbyte(s23.x, s01.y, sh);
            const uint32_t s2 = __builtin_amdgcn_alignbyte(s23.y, s23.x, sh);
            const uint32_t s3 = __builtin_amdgcn_alignbyte(s4, s23.y, sh);
            const float d = half_bits_to_float_fast(s4 >> (8 * sh));
            i32x4 D[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const int ip = c >> 1, pt = c & 1;
                uint32_t b[4];
#pragma unroll
                for (int k = 0; k < 2; k++) {
                    const uint32_t hq = qh[ip][k];
                    const uint32_t h_lo = (pt == 0 ? hq << 4 : hq << 2) & 0x30303030u;
                    const uint32_t h_hi = (pt == 0 ? hq : hq >> 2) & 0x30303030u;
                    b[k] = (ql[c][k] & 0x0F0F0F0Fu) | h_lo;
                    b[2 + k] = ((ql[c][k] >> 4) & 0x0F0F0F0Fu) | h_hi;
                }
                const i32x4 B = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
                D[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[c], B, zero4, 0, 0, 0);
            }
            // scale of quarter g in chunk c: byte 8 ip + 2 part + 4 hs + hh
            const uint32_t slo = hs ? s1 : s0, shi = hs ? s3 : s2;
            float v = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t sw = (c >> 1) ? shi : slo;
                const int scv = (int)(int8_t)((sw >> (8 * (hh + 2 * (c & 1)))) & 0xFFu);
                // exact in int32: |D_p| <= 64 x 63 x 128, |cc| < 2^24
                const int lo = D[c][0] + 256 * D[c][1] - cc[c][0];
                const int hi = D[c][2] + 256 * D[c][3] - cc[c][1];
                const float S = fmaf((float)hi, 65536.0f, (float)lo);
                v = fmaf((float)scv, S, v);
            }
            acc = fmaf(v, d * xs, acc);
            if (hf + 2 >= chunks) {  // this wave's last item of the tile
                // quarters g, g ^ 1 (lanes n + 16 g, xor 16): lanes 0..15 and 32..47 keep the pair sums
                acc += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(acc), 0x401F));
                if ((lane & 16) == 0) part[t & 1][sb][lane >> 5][n] = acc;
                acc = 0.0f;
            }
        }
        slot = slot == kQ6Slots - 1 ? 0 : slot + 1;
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (tiles >= 1 && wv == (tiles - 1) % kQ6Waves && lane < 16) {
        float s = 0.0f;
        for (int k = 0; k < min(nsb, kQ6Waves); k++)
            s += part[(tiles - 1) & 1][k][0][lane] + part[(tiles - 1) & 1][k][1][lane];
        const int row = (tiles - 1) * kQ6TileRows + lane;
        if (row < nr) yout[row] = s;
    }
    __syncthreads();
    for (int r = threadIdx.x; r < nr; r += kQ6Threads) y[r0 + r] = yout[r];
}

bool q6k_mfma_supported(int64_t row_bytes, int64_t cols, int64_t rows, const void *w, const float *x) {
    const int v = tuning().gemv_variant;
    if (v == 1 || v == 4) return false;  // the fp32 kernel stays selectable
    if (cols <= 0 || cols % kQK != 0) return false;
    const int64_t nsb = cols / kQK;
    if (nsb % kQ6HalfSb != 0 || nsb > kQ6MaxSbLds) return false;  // whole items; x fits LDS
    if (row_bytes != nsb * kQ6SbBytes || rows < 1) return false;
    if (((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15u) != 0) return false;
    return (int64_t)kQ6MaxRows * row_bytes < ((int64_t)1 << 31);
}

hipError_t launch_gemv_q6k_mfma(const uint8_t *w, int64_t row_bytes, int64_t cols, const float *x, float *y,
                                int64_t rows, hipStream_t stream) {
    const int64_t cus = device_cus();
    // one workgroup per CU, at most kQ6MaxRows rows each, at least one tile each
    int64_t grid = (rows + kQ6TileRows - 1) / kQ6TileRows;
    if (grid > cus) grid = cus;
    int64_t per = (rows + grid - 1) / grid;
    if (per > kQ6MaxRows) per = kQ6MaxRows;
    grid = (rows + per - 1) / per;
    per = (rows + grid - 1) / grid;
    grid = (rows + per - 1) / per;
    const int nsb = (int)(cols / kQK);
    if (nsb <= 2 * kQ6HalfSb)
        hipLaunchKernelGGL(gemv_q6_k_mfma_tile_kernel<false>, dim3((unsigned)grid), dim3(kQ6Threads), 0, stream, w,
                           row_bytes, nsb, x, y, rows, per);
    else
        hipLaunchKernelGGL(gemv_q6_k_mfma_tile_kernel<true>, dim3((unsigned)grid), dim3(kQ6Threads), 0, stream, w,
                           row_bytes, nsb, x, y, rows, per);
    return hipGetLastError();
}

}  // namespace gollek
