// gguf_gemv_mfma.hip -- Q4_K GEMV (decode, M = 1) on the gfx950 matrix cores.
//
// Same value as the reference raw Q4_K mat-vec (RT/GgufQ4RawDot.java:603-674,
// RT/GgufKQuantLayout.java:67-69; RT/ = runner/gguf/gollek-gguf-core/src/main/
// java/tech/kayys/gollek/gguf/runtime/):
//   y[n] = sum_sb sum_j [ (d sc_j) (sum_{i in j} q_i x_i) - (m_j ? dmin m_j : 0) X_j ]
// over the eight 32-element sub-blocks j of every superblock, X_j = sum of x
// over sub-block j.  Tolerance parity (rel_err <= 1e-3, and within twice the
// reference's own fp32 error for K <= 4096).
//
// Three kernels, by shape:
//   * K <= 4096, at most 64 rows per CU (the 8B-class FFN shapes):
//     gemv_mfma_col_kernel, one superblock column per wave, the
//     workgroup's share in LDS;
//   * K <= 4096, more rows (lm_head): gemv_q4_k_mfma_tile_kernel, 16-row
//     tiles streamed through a shared ring;
//   * K up to 16384: gemv_q4_k_mfma_kernel, per-wave rings of 16 rows x 2
//     superblocks with K split into parts when a workgroup has few tiles.
// All three contract 16 weight rows against 64 columns of x per
// v_mfma_i32_16x16x64_i8, with x as exact integers split into signed-byte
// digit planes (the B operand holds the rows' nibbles as bytes 0..15; A row
// m = 4 h + p holds plane p of sub-block 2 c + h and zeros on the other
// sub-block's columns, so lane n + 16 h of D holds the plane sums of one
// (row, sub-block)).  The K <= 4096 kernels use four planes of 30-bit
// integers (their shared pieces are described further down); the K > 4096
// kernel uses three planes of 22-bit integers:
//
// x (K > 4096).  Per superblock s (256 elements): a power-of-two scale
// xs = 2^(e-22) with max |x| < 2^e, the integers X_i = rint(x_i / xs)
// (|X_i| <= 2^22, so the per-element error is at most 2^-23 of the
// superblock's max |x|) as balanced signed bytes X = 65536 a + 256 b + c
// (c, b in [-128, 127], |a| <= 64), and the sub-block sums xs * sum X_i.
// Built once per workgroup in LDS.  65536 D2 + 256 D1 + D0 = sum q_i X_i
// exactly in int32 (|.| <= 32 * 15 * 2^22 < 2^31).
//
// A records (K > 4096).  Per (superblock, chunk) 208 bytes: for run
// g = 0..3 and plane p = 0..2 the 16 digit bytes of chunk columns
// 16 g .. 16 g + 15, then 16 zero bytes.  Lane (m, g) reads record +
// (3 g + p) * 16 when its A row is live for run g (m < 8, p = m % 4 < 3,
// h = m / 4 = g / 2) and the zero bytes otherwise, so no lane selects or
// masks.  B lane n + 16 g holds 16 nibbles of row n from run g, i.e. chunk
// columns 16 g .. 16 g + 15, low nibbles for g < 2, high for g >= 2.
//
// Streaming (K > 4096).  A workgroup (one per CU) owns an equal share of the
// rows, cut into 16-row tiles; a tile's columns are split into ks K-parts
// when there are fewer tiles than waves.  (tile, K-part) items go
// round-robin to the eight waves.  Each wave streams its items through a
// ring of NSLOT LDS stages of 16 rows x 2 superblocks (rows at a 304-byte
// pitch, so the 16 rows' 16-byte reads fall on distinct banks), filled by
// buffer->LDS loads of whole kilobytes whose row and column masks are folded
// into the offsets.  K-part sums meet in LDS and are added in K order.
#include <type_traits>

#include "gguf_dot4.hpp"
#include "gguf_kernels.hpp"
#include "gguf_mfma_q4k.hpp"

namespace gollek {

using namespace mfq;

namespace {

constexpr int kMfWaves = 8;                       // waves per workgroup
constexpr int kMfThreads = kMfWaves * 64;
constexpr int kTileRows = 16;                     // weight rows per MFMA tile
constexpr int kSps = 2;                           // superblocks per ring stage
// K > 4096 ring stages of Q4_K (144-byte superblocks, quants at 16) or
// Q5_K (176 bytes: qh[32] at 16, quants at 48): kSps superblocks of 16 rows
// at a pitch of an odd number of 16-byte units (304 / 368 bytes), so the 16
// rows' 16-byte reads of one superblock fall on distinct banks.
template <int TYPE>
struct WkGeom {
    static constexpr int PB = TYPE == kQ5_K ? kQ5KBlockBytes : kQKBlockBytes;
    static constexpr int kQOff = TYPE == kQ5_K ? 48 : 16;
    static constexpr int kStageCols = kSps * PB;                          // bytes of a row per stage
    static constexpr int kRowPitch = kStageCols + 16;                     // LDS pitch of a staged row
    static constexpr int kStageDma = (kTileRows * kRowPitch + 1023) / 1024;  // 1 KB loads per stage
    static constexpr int kSlotBytes = kStageDma * 1024;
    static_assert((kRowPitch / 16) % 2 == 1, "odd pitch in 16-byte units");
};
constexpr int kRecBytes = 208;                    // A record of one 64-column chunk
constexpr int kRecZero = 192;                     // offset of its zero bytes
constexpr int kSbRecBytes = 4 * kRecBytes;        // A records of one superblock
constexpr int kMaxParts = 1024;                   // K-part row sums per workgroup

// A records, sub-block sums (xsum[8 sb + 4 h + c] for sub-block 2 c + h) and
// scales of superblocks [0, nsb_pad); superblocks past nsb are zero.  Thread
// t of the workgroup converted float4 t + i * kMfThreads of x, so wave w holds
// superblock w + 8 i in lane order.  Every lane of every wave must call this.
template <int XL>
__device__ __forceinline__ void store_x_records(const XPart<XL> &xp, int nsb, int nsb_pad,
                                                uint8_t *xa, float *xsum, float *xsc) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int i = 0; i < XL; i++) {
        const int sb = (int)(threadIdx.x >> 6) + i * kMfWaves;  // wave-uniform
        const bool live = sb < nsb;
        const float v[4] = {live ? xp.v[i].x : 0.0f, live ? xp.v[i].y : 0.0f,
                            live ? xp.v[i].z : 0.0f, live ? xp.v[i].w : 0.0f};
        uint32_t mb = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) mb = max(mb, __float_as_uint(v[k]) & 0x7FFFFFFFu);
        mb = wave_max_u32(mb);  // NaN and inf order above every finite |x|
        const bool finite = mb < 0x7F800000u;
        int e = 0;
        (void)frexpf(__uint_as_float(mb), &e);  // max |x| < 2^e
        uint32_t w0 = 0, w1 = 0, w2 = 0;
        int s = 0;
#pragma unroll
        for (int k = 0; k < 4; k++) {
            // round to nearest: |X| <= 2^22, so the top digit is at most 64
            // and sum q X over a sub-block stays below 2^31
            const int X = finite ? (int)rintf(ldexpf(v[k], 22 - e)) : 0;
            const int c = (int)(int8_t)(X & 0xFF);
            const int X1 = (X - c) >> 8;
            const int b = (int)(int8_t)(X1 & 0xFF);
            const int a = (X1 - b) >> 8;
            w0 |= ((uint32_t)c & 0xFFu) << (8 * k);
            w1 |= ((uint32_t)b & 0xFFu) << (8 * k);
            w2 |= ((uint32_t)a & 0xFFu) << (8 * k);
            s += X;
        }
        s = sum8_i(s);
        const float scale = !live ? 0.0f : finite ? ldexpf(1.0f, e - 22) : __builtin_nanf("");
        if (sb < nsb_pad) {
            // lane l: chunk l / 16, run (l / 4) % 4, bytes 4 (l % 4) .. + 3 of the run
            uint8_t *rec = xa + sb * kSbRecBytes + (lane >> 4) * kRecBytes;
            // Inline asm: the compiler drops the alias scope of some of these
            // stores and would then wait for the ring's buffer->LDS loads
            // before them.  The caller waits for LDS before its barrier.
            const uint32_t pw = (uint32_t)(uintptr_t)(lds_ptr)(rec + 48 * ((lane >> 2) & 3) + 4 * (lane & 3));
            asm volatile(
                "ds_write_b32 %0, %1\n\t"
                "ds_write_b32 %0, %2 offset:16\n\t"
                "ds_write_b32 %0, %3 offset:32"
                :
                : "v"(pw), "v"(w0), "v"(w1), "v"(w2)
                : "memory");
            if ((lane & 15) == 0) *reinterpret_cast<uint4 *>(rec + kRecZero) = make_uint4(0u, 0u, 0u, 0u);
            if ((lane & 7) == 0) {
                const int j = lane >> 3;  // sub-block
                xsum[sb * 8 + (j & 1) * 4 + (j >> 1)] = (float)s * scale;
            }
            if (lane == 0) xsc[sb] = scale;
        }
    }
}

// Reads one ring stage: the two superblock headers of row n and this lane's
// 16 quant bytes of each of the 2 x 4 chunks.  Inline asm because the
// compiler cannot tell which buffer->LDS load wrote which bytes and would
// wait for all of them; the stage is complete once the VM loads issued after
// it are the only ones outstanding, and the LDS reads finish before the slot
// is refilled.
template <int OFF, int VM, int PB = kQKBlockBytes>
__device__ __forceinline__ void read_stage(uint32_t a_hdr, uint32_t a_qs, u32x4 (&hd)[2],
                                           u32x4 (&q)[2][4]) {
    asm volatile(
        "s_waitcnt vmcnt(%12)\n\t"
        "ds_read_b128 %0, %10 offset:%13\n\t"
        "ds_read_b128 %1, %10 offset:%14\n\t"
        "ds_read_b128 %2, %11 offset:%13\n\t"
        "ds_read_b128 %3, %11 offset:%15\n\t"
        "ds_read_b128 %4, %11 offset:%16\n\t"
        "ds_read_b128 %5, %11 offset:%17\n\t"
        "ds_read_b128 %6, %11 offset:%14\n\t"
        "ds_read_b128 %7, %11 offset:%18\n\t"
        "ds_read_b128 %8, %11 offset:%19\n\t"
        "ds_read_b128 %9, %11 offset:%20\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(hd[0]), "=&v"(hd[1]), "=&v"(q[0][0]), "=&v"(q[0][1]), "=&v"(q[0][2]),
          "=&v"(q[0][3]), "=&v"(q[1][0]), "=&v"(q[1][1]), "=&v"(q[1][2]), "=&v"(q[1][3])
        : "v"(a_hdr), "v"(a_qs), "n"(VM), "n"(OFF), "n"(OFF + PB), "n"(OFF + 32),
          "n"(OFF + 64), "n"(OFF + 96), "n"(OFF + PB + 32),
          "n"(OFF + PB + 64), "n"(OFF + PB + 96)
        : "memory");
}

// Q5_K: read_stage plus this lane's 16 qh bytes of both superblocks (a_qh =
// row n's qh + 16 (g & 1)), under the same wait.
template <int OFF, int VM, int PB>
__device__ __forceinline__ void read_stage5(uint32_t a_hdr, uint32_t a_qs, uint32_t a_qh, u32x4 (&hd)[2],
                                            u32x4 (&q)[2][4], u32x4 (&qh)[2]) {
    asm volatile(
        "s_waitcnt vmcnt(%15)\n\t"
        "ds_read_b128 %0, %12 offset:%16\n\t"
        "ds_read_b128 %1, %12 offset:%17\n\t"
        "ds_read_b128 %2, %13 offset:%16\n\t"
        "ds_read_b128 %3, %13 offset:%18\n\t"
        "ds_read_b128 %4, %13 offset:%19\n\t"
        "ds_read_b128 %5, %13 offset:%20\n\t"
        "ds_read_b128 %6, %13 offset:%17\n\t"
        "ds_read_b128 %7, %13 offset:%21\n\t"
        "ds_read_b128 %8, %13 offset:%22\n\t"
        "ds_read_b128 %9, %13 offset:%23\n\t"
        "ds_read_b128 %10, %14 offset:%16\n\t"
        "ds_read_b128 %11, %14 offset:%17\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(hd[0]), "=&v"(hd[1]), "=&v"(q[0][0]), "=&v"(q[0][1]), "=&v"(q[0][2]), "=&v"(q[0][3]),
          "=&v"(q[1][0]), "=&v"(q[1][1]), "=&v"(q[1][2]), "=&v"(q[1][3]), "=&v"(qh[0]), "=&v"(qh[1])
        : "v"(a_hdr), "v"(a_qs), "v"(a_qh), "n"(VM), "n"(OFF), "n"(OFF + PB), "n"(OFF + 32), "n"(OFF + 64),
          "n"(OFF + 96), "n"(OFF + PB + 32), "n"(OFF + PB + 64), "n"(OFF + PB + 96)
        : "memory");
}

// Position of a wave's stage in its item sequence (wave-uniform counters).
struct StagePos {
    int j = 0;   // item ordinal of the wave (item = wave + 8 j)
    int st = 0;  // stage within the item
    __device__ __forceinline__ void advance(int L) {
        if (++st == L) {
            st = 0;
            ++j;
        }
    }
};

}  // namespace

// TYPE: Q4_K or Q5_K; NSLOT ring stages per wave; MAXSB = superblocks per
// row the LDS tables hold.
template <int TYPE, int NSLOT, int MAXSB>
__global__ __launch_bounds__(kMfThreads) void gemv_q4_k_mfma_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes64, int nsb, const float *__restrict__ x,
    float *__restrict__ y, int64_t rows, int64_t rows_per_wg, int ks) {
    using WG = WkGeom<TYPE>;
    constexpr int kStageCols = WG::kStageCols, kRowPitch = WG::kRowPitch, kStageDma = WG::kStageDma;
    constexpr int kSlotBytes = WG::kSlotBytes;
    constexpr bool Q5 = TYPE == kQ5_K;
    constexpr int XL = (64 * MAXSB + kMfThreads - 1) / kMfThreads;
    // x tables and row sums in one LDS array, the ring in another (the ring's
    // buffer->LDS loads then provably touch none of the tables).
    constexpr int kXsumOff = MAXSB * kSbRecBytes;
    constexpr int kXscOff = kXsumOff + MAXSB * 8 * 4;
    constexpr int kPartsOff = kXscOff + MAXSB * 4;
    __shared__ __attribute__((aligned(16))) uint8_t tabs[kPartsOff + kMaxParts * 4];
    __shared__ __attribute__((aligned(16))) uint8_t ring[kMfWaves * NSLOT * kSlotBytes];
    uint8_t *xa = tabs;
    float *xsum = reinterpret_cast<float *>(tabs + kXsumOff);
    float *xsc = reinterpret_cast<float *>(tabs + kXscOff);
    float *parts = reinterpret_cast<float *>(tabs + kPartsOff);

    const uint32_t row_bytes = (uint32_t)row_bytes64;
    const int lane = threadIdx.x & 63;
    const int wib = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_wg;
    const int nr = (int)(rows - r0 < rows_per_wg ? rows - r0 : rows_per_wg);  // >= 1
    const int tiles = (nr + kTileRows - 1) / kTileRows;
    const int nst = (nsb + kSps - 1) / kSps;
    const int L = nst / ks;  // stages per item (the host picks ks | nst)
    const int items = tiles * ks;
    const int my_items = wib < items ? (items - wib + kMfWaves - 1) / kMfWaves : 0;
    const int total = my_items * L;
    // The host keeps rows_per_wg * row_bytes < 2^31; rows past the workgroup's
    // share are out of the descriptor's range and read as zeros.
    const __amdgpu_buffer_rsrc_t rs = wave_buffer(w + r0 * row_bytes64, (uint32_t)nr * row_bytes);
    uint8_t *myring = ring + wib * (NSLOT * kSlotBytes);

    // Lane l of load k moves staged byte b = 1024 k + 16 l: row b / pitch,
    // column b % pitch (columns past the stage are padding).
    uint32_t dbase[kStageDma];
    uint32_t dcol[kStageDma];
#pragma unroll
    for (int k = 0; k < kStageDma; k++) {
        const uint32_t b = 1024u * k + 16u * lane;
        const uint32_t r = b / kRowPitch, col = b - r * kRowPitch;
        const bool ok = r < (uint32_t)kTileRows && col < (uint32_t)kStageCols;
        dbase[k] = ok ? r * row_bytes + col : kMaskedOffset;
        dcol[k] = ok ? col : 0x40000000u;
    }
    auto issue = [&](uint8_t *slot, const StagePos &p) {
        uint32_t uoff = 0, lim = 0;  // lim = 0 masks every lane
        if (p.j < my_items) {
            const int item = wib + p.j * kMfWaves;
            const int tile = item / ks, kp = item - tile * ks;
            const int sg = kp * L + p.st;
            uoff = (uint32_t)tile * kTileRows * row_bytes + (uint32_t)sg * kStageCols;
            const int left = nsb - sg * kSps;
            lim = (uint32_t)(left < kSps ? left : kSps) * WG::PB;
        }
        uoff = __builtin_amdgcn_readfirstlane(uoff);
        lim = __builtin_amdgcn_readfirstlane(lim);
#pragma unroll
        for (int k = 0; k < kStageDma; k++) {
            const uint32_t o = dcol[k] < lim ? dbase[k] + uoff : kMaskedOffset;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(slot + 1024 * k), 16, o, 0, 0,
                                                     kStreamLoad);
        }
    };

    XPart<XL> xp;
    load_x_parts<kMfThreads, XL>(xp, x, nsb * 8);
    __builtin_amdgcn_sched_barrier(0);  // every x load ahead of the ring loads
    StagePos pf;
#pragma unroll
    for (int j = 0; j < NSLOT; j++) {
        issue(myring + j * kSlotBytes, pf);
        pf.advance(L);
    }
    store_x_records<XL>(xp, nsb, nst * kSps, xa, xsum, xsc);
    // LDS-only exchange: no wait on the ring loads still in flight.
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();

    const int n = lane & 15, g = lane >> 4, h = g & 1;
    const int a_off = (n < 8 && (n & 3) < 3 && (n >> 2) == (g >> 1)) ? (3 * g + (n & 3)) * 16 : kRecZero;
    const int sh = 4 * (g >> 1);
    const uint32_t a_hdr = (uint32_t)(uintptr_t)(lds_ptr)myring + n * kRowPitch;
    const uint32_t a_qs = a_hdr + WG::kQOff + 16 * (g & 1);
    const uint32_t a_qh = a_hdr + 16 + 16 * (g & 1);  // Q5_K's high bits
    const i32x4 zero = {0, 0, 0, 0};

    StagePos cp;
    float acc = 0.0f;
    // One ring stage at slot J (a compile-time slot, so its LDS offsets are
    // instruction immediates).
    auto stage = [&](int q, auto slot_tag) {
        constexpr int J = decltype(slot_tag)::value;
        u32x4 hd[2], qv[2][4], qh[2];
        if constexpr (Q5)
            read_stage5<J * kSlotBytes, kStageDma * (NSLOT - 1), WG::PB>(a_hdr, a_qs, a_qh, hd, qv, qh);
        else
            read_stage<J * kSlotBytes, kStageDma * (NSLOT - 1)>(a_hdr, a_qs, hd, qv);
        issue(myring + J * kSlotBytes, pf);
        pf.advance(L);
        if (q >= total) return;
        const int item = wib + cp.j * kMfWaves;
        const int tile = item / ks, kp = item - tile * ks;
        const int sg = kp * L + cp.st;
#pragma unroll
        for (int s2 = 0; s2 < kSps; s2++) {
            const int sb = sg * kSps + s2;
            const uint8_t *rec = xa + sb * kSbRecBytes + a_off;
            i32x4 A[4];
#pragma unroll
            for (int c = 0; c < 4; c++) A[c] = *reinterpret_cast<const i32x4 *>(rec + c * kRecBytes);
            const float4 xs4 = *reinterpret_cast<const float4 *>(xsum + sb * 8 + 4 * h);
            const float xs = xsc[sb];
            const u32x4 hv = hd[s2];
            const float d = half_bits_to_float_fast(hv.x);
            const float dmin = half_bits_to_float_fast(hv.x >> 16);
            // 6-bit codes of sub-blocks 0-3 and 4-7 (RT/GgufKQuantLayout.java:37-49),
            // shifted so bytes 0 and 2 are this lane's sub-blocks 2 c + h.
            const uint32_t sc03 = (hv.y & 0x3F3F3F3Fu) >> (8 * h);
            const uint32_t mn03 = (hv.z & 0x3F3F3F3Fu) >> (8 * h);
            const uint32_t sc47 = ((hv.w & 0x0F0F0F0Fu) | ((hv.y >> 2) & 0x30303030u)) >> (8 * h);
            const uint32_t mn47 =
                (((hv.w >> 4) & 0x0F0F0F0Fu) | ((hv.z >> 2) & 0x30303030u)) >> (8 * h);
            const float scf[4] = {(float)(sc03 & 0xFFu), (float)((sc03 >> 16) & 0xFFu),
                                  (float)(sc47 & 0xFFu), (float)((sc47 >> 16) & 0xFFu)};
            const float mnf[4] = {(float)(mn03 & 0xFFu), (float)((mn03 >> 16) & 0xFFu),
                                  (float)(mn47 & 0xFFu), (float)((mn47 >> 16) & 0xFFu)};
            float acc_sb = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const u32x4 wq = qv[s2][c];
                i32x4 B = {(int)((wq.x >> sh) & 0x0F0F0F0Fu), (int)((wq.y >> sh) & 0x0F0F0F0Fu),
                           (int)((wq.z >> sh) & 0x0F0F0F0Fu), (int)((wq.w >> sh) & 0x0F0F0F0Fu)};
                if constexpr (Q5) {
                    // element e's fifth bit: qh byte e % 32 (this lane's 16), bit e / 32
                    // = 2 c for the low nibbles (g < 2), 2 c + 1 for the high ones
                    const int hb = 2 * c + (g >> 1);
                    const u32x4 hq = qh[s2];
                    B[0] |= (int)(((hq.x >> hb) & 0x01010101u) << 4);
                    B[1] |= (int)(((hq.y >> hb) & 0x01010101u) << 4);
                    B[2] |= (int)(((hq.z >> hb) & 0x01010101u) << 4);
                    B[3] |= (int)(((hq.w >> hb) & 0x01010101u) << 4);
                }
                const i32x4 D = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[c], B, zero, 0, 0, 0);
                float Sf;
                if constexpr (Q5) {
                    // |sum q X| <= 32 x 31 x 2^22 does not fit int32: the planes
                    // 0, 1 combine exactly, plane 2 joins in one fp32 rounding
                    Sf = fmaf((float)D[2], 65536.0f, (float)(D[0] + 256 * D[1]));
                } else {
                    // |.| <= 32 x 15 x 2^22 < 2^31: exact in int32
                    Sf = (float)(int)((uint32_t)D[0] + ((uint32_t)D[1] << 8) + ((uint32_t)D[2] << 16));
                }
                acc_sb = fmaf(d * scf[c], Sf, acc_sb);
            }
            // min term: zero codes contribute nothing even for a NaN or
            // infinite dmin (minContribution, RT/GgufKQuantLayout.java:67-69)
            const float xsv[4] = {xs4.x, xs4.y, xs4.z, xs4.w};
            float mm = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) mm = fmaf(mnf[c] != 0.0f ? dmin * mnf[c] : 0.0f, xsv[c], mm);
            acc = fmaf(xs, acc_sb, acc) - mm;
        }
        if (cp.st == L - 1) {
            // lanes n and n + 16 hold sub-blocks 2 c and 2 c + 1 of row n
            const float other = __shfl_down(acc, 16, 64);
            const int row = tile * kTileRows + n;
            if (lane < 16 && row < nr) parts[kp * nr + row] = acc + other;
            acc = 0.0f;
        }
        cp.advance(L);
    };
    for (int q0 = 0; q0 < total; q0 += NSLOT) {
        stage(q0, std::integral_constant<int, 0>{});
        stage(q0 + 1, std::integral_constant<int, 1>{});
        if constexpr (NSLOT > 2) stage(q0 + 2, std::integral_constant<int, 2>{});
    }
    // Drain the (masked) ring loads before the workgroup's LDS is released.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    for (int r = threadIdx.x; r < nr; r += kMfThreads) {
        float s = parts[r];
        for (int kp = 1; kp < ks; kp++) s += parts[kp * nr + r];
        y[r0 + r] = s;
    }
}

namespace {

// Q5_K: header (a_hdr = row n's superblock), high-bit bytes 8 g .. 8 g + 7
// (a_qh = a_hdr + 16 + 8 g) and quant bytes (a_q = a_hdr + 48 + 8 g) of one tile.
__device__ __forceinline__ void read_tile_superblock5(uint32_t a_hdr, uint32_t a_qh, uint32_t a_q,
                                                      u32x4 &hv, uint2 &qh, uint2 (&q)[4]) {
    asm volatile(
        "ds_read_b128 %0, %6\n\t"
        "ds_read_b64 %1, %7\n\t"
        "ds_read_b64 %2, %8\n\t"
        "ds_read_b64 %3, %8 offset:32\n\t"
        "ds_read_b64 %4, %8 offset:64\n\t"
        "ds_read_b64 %5, %8 offset:96\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(hv), "=&v"(qh), "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3])
        : "v"(a_hdr), "v"(a_qh), "v"(a_q)
        : "memory");
}

// Q4_0 / Q8_0 on the K <= 4096 kernels: a 256-element piece of a row is
// eight blocks of 32 (block j at BB j: fp16 d, then 16 bytes of nibbles --
// byte i holds element i low and element 16 + i high -- or 32 int8), and
// sub-block j of the Q4_K layout is block j.  B lane n + 16 g of chunk c
// holds the codes of elements 8 g .. 8 g + 7 of blocks 2 c and 2 c + 1
// (Q4_0: the low nibbles of quant bytes 8 (g & 1) .. + 7 for g < 2, their
// high nibbles for g >= 2; Q8_0: quant bytes 8 g .. 8 g + 7), which pair
// with the A rows of x_operands4.  The quant bytes of the even block start
// 2 bytes past a dword, so a lane reads the three dwords covering them and
// realigns; those of the odd block are dword aligned.
//
// Reads one tile's piece of row n (a_q = the row's piece + 8 (g & 1) for
// Q4_0, + 8 g for Q8_0; a_d = the row's piece + BB h): raw[5 c .. 5 c + 2]
// = dwords 2 c BB + {0, 4, 8}, raw[5 c + 3, 5 c + 4] = dwords (2 c + 1) BB +
// 2 + {0, 4} past a_q; dh[c] = the fp16 d of block 2 c + h.
template <int BB>
__device__ __forceinline__ void read_tile_piece32(uint32_t a_q, uint32_t a_d, uint32_t (&raw)[20],
                                                  uint32_t (&dh)[4]) {
#define GOLLEK_OFFS(c) (2 * (c) * BB) / 4, (2 * (c) * BB) / 4 + 1, (2 * (c) * BB) / 4 + 2, \
                       ((2 * (c) + 1) * BB + 2) / 4, ((2 * (c) + 1) * BB + 2) / 4 + 1
    constexpr int o[20] = {GOLLEK_OFFS(0), GOLLEK_OFFS(1), GOLLEK_OFFS(2), GOLLEK_OFFS(3)};
#undef GOLLEK_OFFS
    static_assert(o[19] < 256, "ds_read2 dword offsets");
    uint2 v[10];
    asm volatile(
        "ds_read2_b32 %0, %14 offset0:%16 offset1:%17\n\t"
        "ds_read2_b32 %1, %14 offset0:%18 offset1:%19\n\t"
        "ds_read2_b32 %2, %14 offset0:%20 offset1:%21\n\t"
        "ds_read2_b32 %3, %14 offset0:%22 offset1:%23\n\t"
        "ds_read2_b32 %4, %14 offset0:%24 offset1:%25\n\t"
        "ds_read2_b32 %5, %14 offset0:%26 offset1:%27\n\t"
        "ds_read2_b32 %6, %14 offset0:%28 offset1:%29\n\t"
        "ds_read2_b32 %7, %14 offset0:%30 offset1:%31\n\t"
        "ds_read2_b32 %8, %14 offset0:%32 offset1:%33\n\t"
        "ds_read2_b32 %9, %14 offset0:%34 offset1:%35\n\t"
        "ds_read_u16 %10, %15\n\t"
        "ds_read_u16 %11, %15 offset:%36\n\t"
        "ds_read_u16 %12, %15 offset:%37\n\t"
        "ds_read_u16 %13, %15 offset:%38\n\t"
        "s_waitcnt lgkmcnt(0)"
        : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]), "=&v"(v[6]),
          "=&v"(v[7]), "=&v"(v[8]), "=&v"(v[9]), "=&v"(dh[0]), "=&v"(dh[1]), "=&v"(dh[2]), "=&v"(dh[3])
        : "v"(a_q), "v"(a_d), "n"(o[0]), "n"(o[1]), "n"(o[2]), "n"(o[3]), "n"(o[4]), "n"(o[5]), "n"(o[6]),
          "n"(o[7]), "n"(o[8]), "n"(o[9]), "n"(o[10]), "n"(o[11]), "n"(o[12]), "n"(o[13]), "n"(o[14]),
          "n"(o[15]), "n"(o[16]), "n"(o[17]), "n"(o[18]), "n"(o[19]), "n"(2 * BB), "n"(4 * BB), "n"(6 * BB)
        : "memory");
#pragma unroll
    for (int i = 0; i < 10; i++) {
        raw[2 * i] = v[i].x;
        raw[2 * i + 1] = v[i].y;
    }
}

// The piece's share of row n from blocks 2 c + h (lane n + 16 h, h < 2;
// lanes 32..63 return values of the zero A rows).  Q4_0 codes are stored
// as q + 8 (RT/GgufQ4RawDot.java): the B bytes are q - 8 as signed bytes,
// ((q + 0x78) ^ 0x80) per byte (q + 0x78 <= 0x87, so nothing carries into
// the next byte), and each plane sum is sum (q - 8) X exactly in int32.
template <int TYPE>
__device__ __forceinline__ float q32_tile_piece(const uint32_t (&raw)[20], const uint32_t (&dh)[4],
                                                const XOps4 &o) {
    const int lane = threadIdx.x & 63;
    const uint32_t sh = TYPE == kQ4_0 ? 4u * (uint32_t)(lane >> 5) : 0u;
    const i32x4 zero = {0, 0, 0, 0};
    i32x4 D[4];
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const uint32_t *r = raw + 5 * c;
        const uint32_t l0 = __builtin_amdgcn_alignbyte(r[1], r[0], 2);
        const uint32_t l1 = __builtin_amdgcn_alignbyte(r[2], r[1], 2);
        i32x4 B;
        if constexpr (TYPE == kQ4_0) {
            auto sq = [&](uint32_t v) { return (int)((((v >> sh) & 0x0F0F0F0Fu) + 0x78787878u) ^ 0x80808080u); };
            B = i32x4{sq(l0), sq(l1), sq(r[3]), sq(r[4])};
        } else
            B = i32x4{(int)l0, (int)l1, (int)r[3], (int)r[4]};
        D[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(o.A[c], B, zero, 0, 0, 0);
    }
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; c++) {
        const int d0 = D[c][0], d1 = D[c][1], d2 = D[c][2], d3 = D[c][3];
        // |d0 + 256 d1| < 2^28 (Q8_0) or 2^24 (Q4_0): at most one rounding each
        const float S = fmaf((float)(d2 + 256 * d3), 65536.0f, (float)(d0 + 256 * d1));
        acc = fmaf(half_bits_to_float_fast(dh[c]), S, acc);
    }
    return acc * o.xs;
}

}  // namespace

// ---- K <= 4096: whole 16-row tiles shared by the workgroup -------------
//
// A 16-row tile of a matrix with at most 16 superblocks per row is one
// contiguous block of 16 * row_bytes bytes.  The workgroup (16 waves) streams
// tiles into a shared ring of NSLOT slots (rows at a 2320-byte pitch, so the
// 16 rows' reads of one superblock fall on distinct banks); every wave issues
// an equal share of a tile's 1 KB loads and one barrier per tile publishes
// it.  Per-wave row sums meet in LDS and one wave per tile adds them in
// superblock order.
namespace {

constexpr int kT2Waves = 16;
constexpr int kT2Threads = kT2Waves * 64;
constexpr int kT2Cols = 16 * kQKBlockBytes;                   // 2304
constexpr int kT2Pitch = kT2Cols + 16;                          // 2320
constexpr int kT2Stage = kTileRows * kT2Pitch;                  // 37120
constexpr int kT2Dma = (kT2Stage + 1023) / 1024;                // 37 loads per tile
constexpr int kT2DmaPerWave = (kT2Dma + kT2Waves - 1) / kT2Waves;  // 3
constexpr int kT2Slot = kT2Dma * 1024;
constexpr int kT2MaxRows = 1024;                                // rows per workgroup

}  // namespace

template <int NSLOT>
__global__ __launch_bounds__(kT2Threads) void gemv_q4_k_mfma_tile_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes64, int nsb, const float *__restrict__ x,
    float *__restrict__ y, int64_t rows, int64_t rows_per_wg) {
    static_assert(kT2DmaPerWave * kT2Waves >= kT2Dma, "tile loads");
    static_assert(kT2Waves * 1024 <= kT2Slot, "x scratch fits a slot");
    __shared__ __attribute__((aligned(16))) uint8_t ring[NSLOT * kT2Slot + 1024];  // + sink
    __shared__ float part[2][kT2Waves][32];  // [tile & 1][wave][lane]
    __shared__ float yout[kT2MaxRows];
    // Each wave's x scratch (four digit planes, 1 KB) is kilobyte w of the
    // last ring slot, which the loop first refills after every wave has
    // read its operands back.
    const uint32_t xscr = (uint32_t)(uintptr_t)(lds_ptr)(ring + (NSLOT - 1) * kT2Slot);

    const uint32_t row_bytes = (uint32_t)row_bytes64;
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_wg;
    const int nr = (int)(rows - r0 < rows_per_wg ? rows - r0 : rows_per_wg);  // 1..kT2MaxRows
    const int tiles = (nr + kTileRows - 1) / kTileRows;
    // Rows past the workgroup's share are out of the descriptor's range.
    const __amdgpu_buffer_rsrc_t rs = wave_buffer(w + r0 * row_bytes64, (uint32_t)nr * row_bytes);

    // This wave's tile loads: load k = wv + 16 i moves staged bytes 1024 k + 16 lane
    // (row b / pitch, column b % pitch); loads past the tile write the sink.
    uint32_t dbase[kT2DmaPerWave];
#pragma unroll
    for (int i = 0; i < kT2DmaPerWave; i++) {
        const uint32_t k = (uint32_t)(wv + kT2Waves * i);
        const uint32_t b = 1024u * k + 16u * lane;
        const uint32_t r = b / kT2Pitch, col = b - r * kT2Pitch;
        dbase[i] = (k < (uint32_t)kT2Dma && r < (uint32_t)kTileRows && col < row_bytes) ? r * row_bytes + col
                                                                                       : kMaskedOffset;
    }
    auto issue = [&](int slot, int tile) {
        const uint32_t uoff = tile < tiles ? (uint32_t)tile * kTileRows * row_bytes : kMaskedOffset;
#pragma unroll
        for (int i = 0; i < kT2DmaPerWave; i++) {
            const int k = wv + kT2Waves * i;
            uint8_t *dst = k < kT2Dma ? ring + slot * kT2Slot + 1024 * k : ring + NSLOT * kT2Slot;
            const uint32_t o = (dbase[i] != kMaskedOffset && uoff != kMaskedOffset) ? dbase[i] + uoff : kMaskedOffset;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)dst, 16, o, 0, 0, kStreamLoad);
        }
    };

    // Load order: x, then tile 0; the later tiles only once x has arrived.  A
    // tile is usable when all of it has arrived, and the memory system serves
    // requests issued together interleaved, so this head start makes tile 0
    // complete well before tile 1 instead of together with it.  Wave s owns
    // superblock s (lane l converts its elements 4 l .. 4 l + 3); a wave past
    // nsb converts superblock 0 (its operands are never used).
    const int sb = wv;
    const bool active = sb < nsb;  // wave-uniform
    const float4 xv = reinterpret_cast<const float4 *>(x)[64 * (active ? sb : 0) + lane];
    __builtin_amdgcn_sched_barrier(0);
    issue(0, 0);
    float4 xr = xv;  // the conversion stays below the tile loads
    asm volatile("" : "+v"(xr.x), "+v"(xr.y), "+v"(xr.z), "+v"(xr.w));
    XOps4 xo;
    x_operands4(xr, xscr + 1024u * (uint32_t)wv, xo);
#pragma unroll
    for (int j = 1; j < NSLOT - 1; j++) issue(j, j);

    const int n = lane & 15, g = lane >> 4;
    const uint32_t ring_base = (uint32_t)(uintptr_t)(lds_ptr)ring;
    const uint32_t a_h0 = ring_base + n * kT2Pitch + sb * kQKBlockBytes;
    const uint32_t a_q0 = a_h0 + 16 + 8 * g;
    int slot = 0;
    for (int t = 0; t < tiles; t++) {
        // This wave's loads of tile t are done once the later tiles' loads are
        // the only ones outstanding; the barrier makes every wave's visible and
        // ends every wave's reads of the slot refilled below.
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kT2DmaPerWave * (NSLOT - 2)) : "memory");
        if (t >= 1 && wv == (t - 1) % kT2Waves && lane < 16) {
            const float(*pp)[32] = part[(t - 1) & 1];
            float s = 0.0f;
            for (int k = 0; k < nsb; k++) s += pp[k][lane] + pp[k][lane + 16];
            const int row = (t - 1) * kTileRows + lane;
            if (row < nr) yout[row] = s;
        }
        issue(slot == 0 ? NSLOT - 1 : slot - 1, t + NSLOT - 1);
        if (active) {
            u32x4 hv;
            uint2 q[4];
            const uint32_t off = (uint32_t)slot * kT2Slot;
            read_tile_superblock(a_h0 + off, a_q0 + off, hv, q);
            const float v = q4k_tile_superblock4(hv, q, xo);
            if (lane < 32) part[t & 1][wv][lane] = v;
        }
        slot = slot == NSLOT - 1 ? 0 : slot + 1;
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (tiles >= 1 && wv == (tiles - 1) % kT2Waves && lane < 16) {
        const float(*pp)[32] = part[(tiles - 1) & 1];
        float s = 0.0f;
        for (int k = 0; k < nsb; k++) s += pp[k][lane] + pp[k][lane + 16];
        const int row = (tiles - 1) * kTileRows + lane;
        if (row < nr) yout[row] = s;
    }
    __syncthreads();
    for (int r = threadIdx.x; r < nr; r += kT2Threads) y[r0 + r] = yout[r];
}


// ---- K <= 4096, at most 64 rows per workgroup: one column per wave ---------
//
// For matrices of up to 64 rows per CU (K = 4096 and 16384 rows or fewer),
// the workgroup's whole share of the matrix fits in LDS.  Wave w moves its
// superblock column (the 144 bytes of superblock w of each of the
// workgroup's rows, packed at a 144-byte pitch, so 16-row tiles are 2304
// contiguous bytes) into its own LDS region and works through the tiles as
// its own loads complete.  No wave waits for another's data until the row
// sums meet at the end.
//
// Pacing.  A CU accepts only a few tens of kilobytes of loads in flight; a
// wave whose load does not fit stalls at the issue and cannot compute
// meanwhile.  So a wave issues x and tile 0, and the loads of tile t + 1
// only once tile t has arrived (just before working on it): the CU's queue
// then runs tile-major, each wave's tiles arrive spread over the stream, and
// after the last byte only one tile per wave is left.  Measured on MI355X
// against the alternatives (Q4_K 14336 x 4096): two or all four tiles in
// flight per wave, 9.1 / 9.3 us; a shared-tile ring with one barrier per
// tile, 9.0 us; the whole share issued up front with per-tile barriers,
// 9.8 us (its waves only finish issuing after 3-5 us, so every tile's work
// lands after the stream); this kernel, 8.9 us.  Again on the prepared
// layout (this kernel 7.9 us): every load up front 8.2 us, two tiles ahead
// 8.2 us, waves 8..15 (or 12..15) issuing their whole column at once
// 8.5 (8.2) us, two or four columns per wave (8 or 4 waves) 8.2 / 10.5 us.
// A realtime-stamped copy (tile-aligned loads, 7.7 us) shows the waves all
// starting within 0.5 us and their tiles returning in groups of four (one
// wave per SIMD at a time, the order their loads were accepted): median
// last-tile arrival 4.3, 4.8, 5.3 and 6.2 us for waves 0..3, 4..7, 8..11,
// 12..15; the CU takes in ~22 B/ns meanwhile.
namespace {

constexpr int kColWaves = 16;
constexpr int kColThreads = kColWaves * 64;
// x scratch of the wave (four digit planes of a superblock).
constexpr int kColX = 1024;

// A column's region: the rows' PB-byte pieces (Q4_K, Q4_0: a 144-byte
// superblock or eight blocks; Q5_K: 176 bytes; Q8_0: eight 34-byte blocks,
// 272 bytes) packed at a PB-byte pitch in up to 9 KB, then kColX.
template <int TYPE>
struct ColGeom {
    static constexpr int PB = TYPE == kQ8_0 ? 8 * kQ8BlockBytes : TYPE == kQ5_K ? kQ5KBlockBytes : kQKBlockBytes;
    static constexpr int NL = 9;
    static constexpr int kW = NL * 1024;                    // column bytes of a wave
    static constexpr int kRegion = kW + kColX;              // 16 regions: 160 KB
    static constexpr int kMaxTiles = kW / (kTileRows * PB);  // whole tiles only
    static constexpr int kMaxRows = kMaxTiles * kTileRows;   // 64 (Q5_K: 48, Q8_0: 32)
    static constexpr int kTileBytes = kTileRows * PB;
    static_assert(kMaxTiles >= 2 && kMaxTiles <= 4, "up to four tiles");
};

}  // namespace

// TYPE: Q4_K, Q5_K, Q4_0 or Q8_0; a piece is the 256 elements of one
// superblock column.  PREP: w is the prepared layout (prepare_col_layout):
// each workgroup's block of rows stored column by column, so a wave's column
// is one contiguous run of its rows' pieces; the same bytes otherwise.
// Measured on MI355X (Q4_K 14336 x 4096): 7.8 us against 8.8 us reading the
// GGUF rows, whose columns are 144-byte pieces 2304 bytes apart.
//
// Tiles.  Each 16-row tile of a column is moved by its own loads (1 KB
// loads, then 256-byte tails of 4 bytes a lane: 2304 = 2 KB + 256, 2816 =
// 2 KB + 3 x 256, 4352 = 4 KB + 256), so a tile's wait covers exactly its
// bytes, and its row sums go to the first 128 bytes of the tile in LDS once
// it has been read (pair h of row n at float 2 n + h).  Measured against
// 1 KB loads spanning tile boundaries with the row sums in the x scratch:
// Q4_K 14336 x 4096 7.7 against 7.9 us, Q4_0 11008 x 4096 7.4 against
// 7.9 us, Q8_0 4096 x 4096 5.33 against 5.40 us (Q5_K 4.98 against
// 4.92 us: its 768-byte tail takes three loads).
// Also measured and dropped: the first four waves taking the last tile of
// columns 12..15 (whose tiles arrive last), 8.2 us.
//
// NV = 2 .. 4 (the small-M GEMM's M): the second vector's digits sit in A
// rows 8..15, which the single vector leaves zero, so each MFMA serves both
// and output lanes 32..63 hold the second vector's sums; vectors 2 and 3
// take a second operand set (a second MFMA per chunk on the same B).
// Vector v is x + v K, its results y + v rows.  XB: x holds bf16 bit
// patterns (the GEMM's input), widened to fp32 exactly as they load.
template <int TYPE, bool PREP, int NV = 1, bool XB = false>
__global__ __launch_bounds__(kColThreads) void gemv_mfma_col_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes64, int nsb, const float *__restrict__ x,
    float *__restrict__ y, int64_t rows, int rows_per_wg) {
    using G = ColGeom<TYPE>;
    constexpr int PB = G::PB;
    constexpr int TB = G::kTileBytes;
    constexpr int kFull = TB / 1024;          // 1 KB loads per tile
    constexpr int kTail = (TB % 1024) / 256;  // 256-byte tail loads per tile
    static_assert(TB % 256 == 0 && PB % 16 == 0, "tiles are whole loads");
    __shared__ __attribute__((aligned(16))) uint8_t lds[kColWaves * G::kRegion];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_wg;
    const int nr = (int)(rows - r0 < rows_per_wg ? rows - r0 : rows_per_wg);  // 1..kMaxRows
    const uint32_t row_bytes = (uint32_t)row_bytes64;
    const int tiles = (nr + kTileRows - 1) / kTileRows;
    const uint32_t lds0 = (uint32_t)(uintptr_t)(lds_ptr)lds;

    if (wv < nsb) {  // wave-uniform; waves past nsb own no column
        // The column's rows: nr PB-byte pieces (PREP: contiguous from
        // w + r0 row_bytes + nr PB wv; otherwise row r's piece at r row_bytes
        // from w + r0 row_bytes + PB wv, the descriptor ending at the last
        // row's piece: (nr - 1) row_bytes + PB <= nr row_bytes - PB wv).
        const __amdgpu_buffer_rsrc_t rs =
            PREP ? wave_buffer(w + r0 * row_bytes64 + (int64_t)nr * PB * wv, (uint32_t)(nr * PB))
                 : wave_buffer(w + r0 * row_bytes64 + PB * wv, (uint32_t)nr * row_bytes - PB * wv);
        // Byte b of a column: row b / PB, byte b % PB of the row's piece;
        // rows past nr read as zeros.
        auto offset = [&](uint32_t b) {
            const uint32_t r = b / PB, col = b - r * PB;
            return r < (uint32_t)nr ? (PREP ? b : r * row_bytes + col) : kMaskedOffset;
        };
        uint8_t *const region = lds + wv * G::kRegion;
        auto issue = [&](int t) {
            const uint32_t tb = (uint32_t)(TB * t);
#pragma unroll
            for (int j = 0; j < kFull; j++) {
                const uint32_t o = offset(tb + 1024u * j + 16u * lane);  // a named local for the builtin
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(region + tb + 1024 * j), 16, o, 0, 0,
                                                         kStreamLoad);
            }
#pragma unroll
            for (int j = 0; j < kTail; j++) {
                const uint32_t o = offset(tb + 1024u * kFull + 256u * j + 4u * lane);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(region + tb + 1024 * kFull + 256 * j), 4, o,
                                                         0, 0, kStreamLoad);
            }
        };

        // x first, then tile 0, then the digit planes while it flies.  Pacing:
        // each next tile is issued once the previous one has arrived (see
        // above).
        auto load_x = [&](int v) {
            if constexpr (XB) {
                const uint2 u = reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(x) +
                                                                (int64_t)v * nsb * kQK)[64 * wv + lane];
                return float4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u),
                              __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xFFFF0000u)};
            } else {
                return reinterpret_cast<const float4 *>(x + (int64_t)v * nsb * kQK)[64 * wv + lane];
            }
        };
        const float4 xv = load_x(0);
        float4 xv2 = xv, xv3 = xv, xv4 = xv;
        if constexpr (NV >= 2) xv2 = load_x(1);
        if constexpr (NV >= 3) xv3 = load_x(2);
        if constexpr (NV >= 4) xv4 = load_x(3);
        __builtin_amdgcn_sched_barrier(0);
        issue(0);
        __builtin_amdgcn_sched_barrier(0);
        const uint32_t rbase = lds0 + wv * G::kRegion;
        XOps4 xo, xo2;
        float4 xr = xv;  // the conversion stays below the tile's loads
        asm volatile("" : "+v"(xr.x), "+v"(xr.y), "+v"(xr.z), "+v"(xr.w));
        // vectors a (A rows 0..7, output lanes 0..31) and b (rows 8..15,
        // lanes 32..63) in one operand set; b absent: rows 8..15 zero
        auto pair_operands = [&](float4 a, float4 b, bool has_b) {
            asm volatile("" : "+v"(b.x), "+v"(b.y), "+v"(b.z), "+v"(b.w));
            XOpsC c0, c1;
            x_operands4c(a, rbase + G::kW, c0);
            if (!has_b) return x_expand(c0);
            x_operands4c<true>(b, rbase + G::kW, c1);
            const bool second = lane >= 32;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                c0.d[k] = uint2{c0.d[k].x | c1.d[k].x, c0.d[k].y | c1.d[k].y};
                c0.xs4[k] = second ? c1.xs4[k] : c0.xs4[k];
            }
            c0.xs = second ? c1.xs : c0.xs;
            return x_expand(c0);
        };
        if constexpr (NV == 1) {
            x_operands4(xr, rbase + G::kW, xo);
        } else {
            xo = pair_operands(xr, xv2, true);
            if constexpr (NV >= 3) {
                float4 xr3 = xv3;
                asm volatile("" : "+v"(xr3.x), "+v"(xr3.y), "+v"(xr3.z), "+v"(xr3.w));
                xo2 = pair_operands(xr3, xv4, NV == 4);
            }
        }

        const int n = lane & 15, g = lane >> 4;
        for (int t = 0; t < tiles; t++) {
            wait_vm<0>();
            if (t + 1 < tiles) issue(t + 1);
            // Row n's piece of the tile: Q4_K header and quants; Q4_0 / Q8_0
            // quants and scales (see read_tile_piece32).
            const uint32_t a_t = rbase + TB * t;
            const uint32_t a_h = a_t + n * PB;
            float v, v2 = 0.0f;
            if constexpr (TYPE == kQ4_K) {
                u32x4 hv;
                uint2 q[4];
                read_tile_superblock(a_h, a_h + 16 + 8 * g, hv, q);
                v = q4k_tile_superblock4(hv, q, xo);
                if constexpr (NV >= 3) v2 = q4k_tile_superblock4(hv, q, xo2);
            } else if constexpr (TYPE == kQ5_K) {
                u32x4 hv;
                uint2 qh, q[4];
                read_tile_superblock5(a_h, a_h + 16 + 8 * g, a_h + 48 + 8 * g, hv, qh, q);
                v = q4k_tile_superblock4<true>(hv, q, xo, qh);
                if constexpr (NV >= 3) v2 = q4k_tile_superblock4<true>(hv, q, xo2, qh);
            } else {
                uint32_t raw[20], dh[4];
                const uint32_t a_q = a_h + 8 * (TYPE == kQ4_0 ? (g & 1) : g);
                const uint32_t a_d = a_h + (TYPE == kQ8_0 ? kQ8BlockBytes : kQ4BlockBytes) * (g & 1);
                read_tile_piece32<TYPE == kQ8_0 ? kQ8BlockBytes : kQ4BlockBytes>(a_q, a_d, raw, dh);
                v = q32_tile_piece<TYPE>(raw, dh, xo);
                if constexpr (NV >= 3) v2 = q32_tile_piece<TYPE>(raw, dh, xo2);
            }
            // lane n + 16 h: sub-blocks 2 c + h of row n, kept apart until the
            // row sums; the tile has been read (read_* wait for their reads).
            // Vector j's sums at + 128 j (lanes 32..63 hold vectors 1 and 3).
            if (lane < 32) lds_store_f32(a_t + 8 * n + 4 * g, v);
            else if (NV >= 2) lds_store_f32(a_t + 128 + 8 * n + 4 * (g & 1), v);
            if constexpr (NV >= 3) {
                if (lane < 32) lds_store_f32(a_t + 256 + 8 * n + 4 * g, v2);
                else if (NV == 4) lds_store_f32(a_t + 384 + 8 * n + 4 * (g & 1), v2);
            }
        }
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    // Row sums in superblock order (vector v's at + 128 v).
    for (int q = threadIdx.x; q < NV * nr; q += kColThreads) {
        int v = 0, r = q;
        if constexpr (NV > 1) {
            v = q / nr;
            r = q - v * nr;
        }
        const int off = TB * (r >> 4) + 128 * v + 8 * (r & 15);
        float2 p[kColWaves];
#pragma unroll
        for (int k = 0; k < kColWaves; k++)
            p[k] = k < nsb ? *reinterpret_cast<const float2 *>(lds + k * G::kRegion + off) : make_float2(0.0f, 0.0f);
        float s = 0.0f;
#pragma unroll
        for (int k = 0; k < kColWaves; k++) s += p[k].x + p[k].y;
        y[(int64_t)v * rows + r0 + r] = s;
    }
}

// ---- 4096 < K <= 16384, few rows per CU: several columns per wave ----------
//
// The column kernel for wide rows (e.g. Q4_K 4096 x 14336, the FFN down
// projection): a workgroup per CU, its block of at most kMaxRows rows read
// from the same prepared layout (or the GGUF rows), wave w taking the
// superblock columns w, w + 16, ... (up to four).  Its units are (column,
// 16-row tile), column by column, each moved by its own loads (as the column
// kernel's tiles) into two slots of the wave's LDS region with the same
// pacing: unit k + 1 is issued once unit k has arrived.  x: every column's
// superblock is loaded up front and its digit planes built while unit 0's
// loads fly, kept compactly (XOpsC) until the column's units.  Row sums accumulate per wave in LDS (pair h of
// row r at part[w][r][h]) and meet at the end in wave order.
constexpr int kWideMaxCols = 4;  // columns per wave (K <= 16384)

// NV = 2, XB: as the column kernel's (the small-M GEMM's M = 2 on bf16 X):
// the second vector's digits in A rows 8..15 of the same compact operands,
// its sums in output lanes 32..63 and a second row-sum buffer.
template <int TYPE, bool PREP, int NV = 1, bool XB = false>
__global__ __launch_bounds__(kColThreads) void gemv_mfma_wide_kernel(
    const uint8_t *__restrict__ w, int64_t row_bytes64, int nsb, const float *__restrict__ x,
    float *__restrict__ y, int64_t rows, int rows_per_wg) {
    using G = ColGeom<TYPE>;
    constexpr int PB = G::PB;
    constexpr int TB = G::kTileBytes;
    constexpr int kFull = TB / 1024;
    constexpr int kTail = (TB % 1024) / 256;
    constexpr int kRegionW = 2 * TB + kColX;  // two unit slots, then the x scratch
    static_assert(NV == 1 || NV == 2, "one or two vectors");
    __shared__ __attribute__((aligned(16))) uint8_t lds[kColWaves * kRegionW];
    __shared__ float part[NV][kColWaves][G::kMaxRows][2];
    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int64_t r0 = (int64_t)blockIdx.x * rows_per_wg;
    const int nr = (int)(rows - r0 < rows_per_wg ? rows - r0 : rows_per_wg);  // 1..kMaxRows
    const uint32_t row_bytes = (uint32_t)row_bytes64;
    const int tiles = (nr + kTileRows - 1) / kTileRows;
    const int ncol = wv < nsb ? (nsb - wv + kColWaves - 1) / kColWaves : 0;  // wave-uniform
    // superblock c of vector v (XB: bf16 bits widened exactly)
    auto load_x = [&](int v, int c) {
        if constexpr (XB) {
            const uint2 u = reinterpret_cast<const uint2 *>(reinterpret_cast<const uint16_t *>(x) +
                                                            (int64_t)v * nsb * kQK)[64 * c + lane];
            return float4{__uint_as_float(u.x << 16), __uint_as_float(u.x & 0xFFFF0000u),
                          __uint_as_float(u.y << 16), __uint_as_float(u.y & 0xFFFF0000u)};
        } else {
            return reinterpret_cast<const float4 *>(x + (int64_t)v * nsb * kQK)[64 * c + lane];
        }
    };

    if (ncol > 0) {
        // The workgroup's block: nr rows (PREP: column c is nr PB-byte pieces
        // at nr PB c; otherwise row r's piece of column c at r row_bytes + PB c).
        const __amdgpu_buffer_rsrc_t rs = wave_buffer(w + r0 * row_bytes64, (uint32_t)nr * row_bytes);
        auto offset = [&](int c, uint32_t b) {  // byte b of column c
            const uint32_t r = b / PB, col = b - r * PB;
            return r < (uint32_t)nr ? (PREP ? (uint32_t)(nr * PB * c) + b : r * row_bytes + PB * c + col)
                                    : kMaskedOffset;
        };
        uint8_t *const region = lds + wv * kRegionW;
        const uint32_t rbase = (uint32_t)(uintptr_t)(lds_ptr)region;
        const int nunits = ncol * tiles;
        auto issue = [&](int k) {
            const int i = k / tiles, t = k - i * tiles;
            const int c = wv + kColWaves * i;
            const uint32_t tb = (uint32_t)(TB * t);
            uint8_t *const dst = region + TB * (k & 1);
#pragma unroll
            for (int j = 0; j < kFull; j++) {
                const uint32_t o = offset(c, tb + 1024u * j + 16u * lane);  // a named local for the builtin
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(dst + 1024 * j), 16, o, 0, 0, kStreamLoad);
            }
#pragma unroll
            for (int j = 0; j < kTail; j++) {
                const uint32_t o = offset(c, tb + 1024u * kFull + 256u * j + 4u * lane);
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(dst + 1024 * kFull + 256 * j), 4, o, 0, 0,
                                                         kStreamLoad);
            }
        };
        // x of every column (past nsb the wave's first again, unused), then
        // unit 0, then every column's operands while unit 0 flies (built
        // between units instead, they held up the units: 9.3 against 8.0 us
        // for Q4_K 4096 x 14336).
        float4 xq[kWideMaxCols], xq2[kWideMaxCols];
#pragma unroll
        for (int i = 0; i < kWideMaxCols; i++) {
            const int c = wv + kColWaves * i;
            xq[i] = load_x(0, c < nsb ? c : wv);
            if constexpr (NV == 2) xq2[i] = load_x(1, c < nsb ? c : wv);
        }
        __builtin_amdgcn_sched_barrier(0);
        issue(0);
        __builtin_amdgcn_sched_barrier(0);
        XOpsC xc[kWideMaxCols];
#pragma unroll
        for (int i = 0; i < kWideMaxCols; i++) {
            if (i < ncol) {
                x_operands4c(xq[i], rbase + 2 * TB, xc[i]);
                if constexpr (NV == 2) {
                    // the second vector in rows 8..15 of the same registers
                    XOpsC c1;
                    x_operands4c<true>(xq2[i], rbase + 2 * TB, c1);
                    const bool second = lane >= 32;
#pragma unroll
                    for (int k = 0; k < 4; k++) {
                        xc[i].d[k] = uint2{xc[i].d[k].x | c1.d[k].x, xc[i].d[k].y | c1.d[k].y};
                        xc[i].xs4[k] = second ? c1.xs4[k] : xc[i].xs4[k];
                    }
                    xc[i].xs = second ? c1.xs : xc[i].xs;
                }
            }
        }

        const int n = lane & 15, g = lane >> 4;
        float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};  // per tile, summed over the wave's columns in order
        static_assert(G::kMaxTiles <= 4, "four tile sums");
#pragma unroll
        for (int i = 0; i < kWideMaxCols; i++) {  // unrolled: xc[i] stays in registers
            if (i >= ncol) break;
            const XOps4 xo = x_expand(xc[i]);
            for (int t = 0; t < tiles; t++) {
                const int k = i * tiles + t;
                wait_vm<0>();
                if (k + 1 < nunits) issue(k + 1);
                const uint32_t a_h = rbase + TB * (k & 1) + n * PB;
                float v;
                if constexpr (TYPE == kQ4_K) {
                    u32x4 hv;
                    uint2 q[4];
                    read_tile_superblock(a_h, a_h + 16 + 8 * g, hv, q);
                    v = q4k_tile_superblock4(hv, q, xo);
                } else if constexpr (TYPE == kQ5_K) {
                    u32x4 hv;
                    uint2 qh, q[4];
                    read_tile_superblock5(a_h, a_h + 16 + 8 * g, a_h + 48 + 8 * g, hv, qh, q);
                    v = q4k_tile_superblock4<true>(hv, q, xo, qh);
                } else {
                    uint32_t raw[20], dh[4];
                    const uint32_t a_q = a_h + 8 * (TYPE == kQ4_0 ? (g & 1) : g);
                    const uint32_t a_d = a_h + (TYPE == kQ8_0 ? kQ8BlockBytes : kQ4BlockBytes) * (g & 1);
                    read_tile_piece32<TYPE == kQ8_0 ? kQ8BlockBytes : kQ4BlockBytes>(a_q, a_d, raw, dh);
                    v = q32_tile_piece<TYPE>(raw, dh, xo);
                }
                // lane n + 16 h: sub-blocks 2 c + h of row n
#pragma unroll
                for (int j = 0; j < 4; j++) acc[j] += t == j ? v : 0.0f;
            }
        }
        if (lane < 32 || NV == 2)
            for (int t = 0; t < tiles; t++)
                part[lane >> 5][wv][16 * t + n][g & 1] =
                    t == 0 ? acc[0] : t == 1 ? acc[1] : t == 2 ? acc[2] : acc[3];
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const int nw = nsb < kColWaves ? nsb : kColWaves;
    for (int q = threadIdx.x; q < NV * nr; q += kColThreads) {
        int v = 0, r = q;
        if constexpr (NV == 2) {
            v = q >= nr ? 1 : 0;
            r = q - v * nr;
        }
        float s = 0.0f;
        for (int k = 0; k < nw; k++) s += part[v][k][r][0] + part[v][k][r][1];
        y[(int64_t)v * rows + r0 + r] = s;
    }
}

namespace {

struct MfmaPlan {
    int64_t grid = 0, rows_per_wg = 0;
    int ks = 1;
};

MfmaPlan plan_mfma(int64_t rows, int nsb) {
    MfmaPlan p;
    const int64_t cus = device_cus();
    int64_t grid = (rows + kTileRows - 1) / kTileRows;  // at least a tile per workgroup
    if (grid > cus) grid = cus;
    int64_t per = (rows + grid - 1) / grid;
    if (per > kMaxParts) per = kMaxParts;
    grid = (rows + per - 1) / per;
    per = (rows + grid - 1) / grid;
    grid = (rows + per - 1) / per;  // every workgroup gets at least one row
    const int tiles = (int)((per + kTileRows - 1) / kTileRows);
    const int nst = (nsb + kSps - 1) / kSps;
    // K-parts: the divisor of the stage count that minimises the busiest
    // wave's stages (ties to fewer parts), within the LDS row-sum buffer.
    int best = 1;
    int64_t best_cost = INT64_MAX;
    for (int k = 1; k <= nst; k++) {
        if (nst % k != 0 || (int64_t)k * per > kMaxParts) continue;
        const int64_t cost = (((int64_t)tiles * k + kMfWaves - 1) / kMfWaves) * (nst / k);
        if (cost < best_cost) {
            best_cost = cost;
            best = k;
        }
    }
    p.grid = grid;
    p.rows_per_wg = per;
    p.ks = best;
    return p;
}

}  // namespace

bool q4k_mfma_supported(int64_t row_bytes, int64_t cols, int64_t rows, const void *w,
                        const float *x) {
    (void)rows;  // a workgroup's descriptor spans <= kMaxParts rows of <= 64 superblocks
    if (tuning().gemv_variant == 1) return false;
    const int64_t nsb = cols / kQK;
    return nsb >= 1 && nsb <= 64 && row_bytes == nsb * kQKBlockBytes &&
           (reinterpret_cast<uintptr_t>(w) & 15u) == 0 && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

hipError_t launch_gemv_q4k_mfma(const uint8_t *w, int64_t row_bytes, int64_t cols,
                                const float *x, float *y, int64_t rows, hipStream_t stream,
                                const uint8_t *prep, int64_t prep_rows) {
    const int nsb = (int)(cols / kQK);
    const int64_t cus = device_cus();
    // At most 64 rows per CU: one workgroup per CU's block of rows, one
    // superblock column per wave (K <= 4096) or several (the wide kernel,
    // K <= 16384); gemv_variant 3 keeps the shared tiles.
    const int64_t col_rows = col_layout_rows(kQ4_K, rows, cols);
    if (col_rows > 0) {
        const dim3 grid((unsigned)((rows + col_rows - 1) / col_rows));
        const bool use_prep = prep != nullptr && prep_rows == col_rows;
        const uint8_t *src = use_prep ? prep : w;
        if (nsb <= kColWaves) {
            if (use_prep)
                hipLaunchKernelGGL((gemv_mfma_col_kernel<kQ4_K, true>), grid, dim3(kColThreads), 0, stream, src,
                                   row_bytes, nsb, x, y, rows, (int)col_rows);
            else
                hipLaunchKernelGGL((gemv_mfma_col_kernel<kQ4_K, false>), grid, dim3(kColThreads), 0, stream, src,
                                   row_bytes, nsb, x, y, rows, (int)col_rows);
        } else {
            if (use_prep)
                hipLaunchKernelGGL((gemv_mfma_wide_kernel<kQ4_K, true>), grid, dim3(kColThreads), 0, stream, src,
                                   row_bytes, nsb, x, y, rows, (int)col_rows);
            else
                hipLaunchKernelGGL((gemv_mfma_wide_kernel<kQ4_K, false>), grid, dim3(kColThreads), 0, stream, src,
                                   row_bytes, nsb, x, y, rows, (int)col_rows);
        }
        return hipGetLastError();
    }
    if (nsb <= 16) {
        // one workgroup per CU, at most kT2MaxRows rows each, at least one tile each
        int64_t grid = (rows + kTileRows - 1) / kTileRows;
        if (grid > cus) grid = cus;
        int64_t per = (rows + grid - 1) / grid;
        if (per > kT2MaxRows) per = kT2MaxRows;
        grid = (rows + per - 1) / per;
        per = (rows + grid - 1) / grid;
        grid = (rows + per - 1) / per;
        hipLaunchKernelGGL((gemv_q4_k_mfma_tile_kernel<3>), dim3((unsigned)grid), dim3(kT2Threads), 0,
                           stream, w, row_bytes, nsb, x, y, rows, per);
        return hipGetLastError();
    }
    const MfmaPlan p = plan_mfma(rows, nsb);
    hipLaunchKernelGGL((gemv_q4_k_mfma_kernel<kQ4_K, 2, 64>), dim3((unsigned)p.grid), dim3(kMfThreads), 0,
                       stream, w, row_bytes, nsb, x, y, rows, p.rows_per_wg, p.ks);
    return hipGetLastError();
}

// Q5_K past K = 4096 (the column kernel takes K <= 4096): the K > 4096
// Q4_K kernel with the fifth bit from qh.
bool q5k_wide_mfma_supported(int64_t row_bytes, int64_t cols, int64_t rows, const void *w, const float *x) {
    (void)rows;
    const int v = tuning().gemv_variant;
    if (v == 1 || v == 4) return false;  // the fp32 kernel stays selectable
    if (cols <= 0 || cols % kQK != 0) return false;
    const int64_t nsb = cols / kQK;
    return nsb > 16 && nsb <= 64 && row_bytes == nsb * kQ5KBlockBytes &&
           ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15u) == 0;
}

hipError_t launch_gemv_q5k_wide_mfma(const uint8_t *w, int64_t row_bytes, int64_t cols, const float *x, float *y,
                                     int64_t rows, hipStream_t stream) {
    const MfmaPlan p = plan_mfma(rows, (int)(cols / kQK));
    hipLaunchKernelGGL((gemv_q4_k_mfma_kernel<kQ5_K, 2, 64>), dim3((unsigned)p.grid), dim3(kMfThreads), 0,
                       stream, w, row_bytes, (int)(cols / kQK), x, y, rows, p.rows_per_wg, p.ks);
    return hipGetLastError();
}

// Q4_0 / Q8_0 / Q5_K on the matrix cores (the column kernel): K a multiple
// of 256 up to 4096, 16-byte aligned weights, rows and x.  Every row count runs on
// it (workgroups of at most ColGeom<TYPE>::kMaxRows rows, more workgroups
// than CUs when needed), so a row's sum has the same bits whatever the row
// count of the call.
bool q32_mfma_supported(int type_id, int64_t row_bytes, int64_t cols, int64_t rows, const void *w,
                        const float *x) {
    if (type_id != kQ4_0 && type_id != kQ8_0 && type_id != kQ5_K) return false;
    const int v = tuning().gemv_variant;
    if (v == 1 || v == 4) return false;  // fp32 / ring / Q5_K fp32 paths kept selectable
    if (cols <= 0 || cols % kQK != 0 || cols / kQK > 16 * kWideMaxCols || rows <= 0) return false;
    const int64_t piece = type_id == kQ8_0 ? 8 * kQ8BlockBytes : type_id == kQ5_K ? kQ5KBlockBytes : kQKBlockBytes;
    if (row_bytes != cols / kQK * piece || (row_bytes & 15) != 0) return false;
    return ((reinterpret_cast<uintptr_t>(w) | reinterpret_cast<uintptr_t>(x)) & 15u) == 0;
}

// The small-M GEMM at M = 1 .. 4 on the column kernel (X: M bf16 rows of K,
// Y: M rows of N floats): the GEMV's stream of the weights once, two
// vectors in each MFMA; past K = 4096 (up to 16384) the wide kernel, M up
// to 2.  Weights of a type those kernels take, K a multiple of 256, a row
// count their partition takes, 16-byte aligned weights and 8-byte aligned X.
bool gemm_col_supported(int type_id, int64_t row_bytes, int M, int N, int K, const void *w, const void *x) {
    if (M < 1 || M > 4 || N <= 0 || K <= 0 || K % kQK != 0 || K / kQK > kColWaves * kWideMaxCols) return false;
    if (K / kQK > kColWaves && M > 2) return false;  // the wide kernel holds two vectors
    if (type_id != kQ4_K && type_id != kQ5_K && type_id != kQ4_0 && type_id != kQ8_0) return false;
    const int64_t piece = type_id == kQ8_0 ? 8 * kQ8BlockBytes : type_id == kQ5_K ? kQ5KBlockBytes : kQKBlockBytes;
    if (row_bytes != (int64_t)(K / kQK) * piece) return false;
    if ((reinterpret_cast<uintptr_t>(w) & 15u) != 0 || (reinterpret_cast<uintptr_t>(x) & 7u) != 0) return false;
    return col_layout_rows(type_id, N, K) > 0;
}

hipError_t launch_gemm_col(int type_id, const uint8_t *w, int64_t row_bytes, const uint16_t *x, float *y, int M,
                           int N, int K, hipStream_t stream, const uint8_t *prep, int64_t prep_rows) {
    const int nsb = K / kQK;
    const int64_t col_rows = col_layout_rows(type_id, N, K);
    if (col_rows <= 0) return hipErrorInvalidValue;  // callers check gemm_col_supported first
    const bool use_prep = prep != nullptr && prep_rows == col_rows;
    const uint8_t *src = use_prep ? prep : w;
    if (src == nullptr) return hipErrorInvalidValue;  // no GGUF rows and no layout for this partition
    const dim3 grid((unsigned)((N + col_rows - 1) / col_rows));
    const float *xf = reinterpret_cast<const float *>(x);
#define GOLLEK_GEMM_COL_NV(T, NV)                                                                              \
    do {                                                                                                       \
        if (use_prep)                                                                                          \
            hipLaunchKernelGGL((gemv_mfma_col_kernel<T, true, NV, true>), grid, dim3(kColThreads), 0, stream,   \
                               src, row_bytes, nsb, xf, y, (int64_t)N, (int)col_rows);                        \
        else                                                                                                   \
            hipLaunchKernelGGL((gemv_mfma_col_kernel<T, false, NV, true>), grid, dim3(kColThreads), 0, stream,  \
                               src, row_bytes, nsb, xf, y, (int64_t)N, (int)col_rows);                        \
    } while (0)
#define GOLLEK_GEMM_WIDE_NV(T, NV)                                                                             \
    do {                                                                                                       \
        if (use_prep)                                                                                          \
            hipLaunchKernelGGL((gemv_mfma_wide_kernel<T, true, NV, true>), grid, dim3(kColThreads), 0, stream,  \
                               src, row_bytes, nsb, xf, y, (int64_t)N, (int)col_rows);                        \
        else                                                                                                   \
            hipLaunchKernelGGL((gemv_mfma_wide_kernel<T, false, NV, true>), grid, dim3(kColThreads), 0, stream, \
                               src, row_bytes, nsb, xf, y, (int64_t)N, (int)col_rows);                        \
    } while (0)
#define GOLLEK_GEMM_COL(T)                                                                                      \
    do {                                                                                                        \
        if (nsb > kColWaves) {                                                                                  \
            if (M == 1) GOLLEK_GEMM_WIDE_NV(T, 1);                                                              \
            else GOLLEK_GEMM_WIDE_NV(T, 2);                                                                     \
        } else if (M == 1) GOLLEK_GEMM_COL_NV(T, 1);                                                            \
        else if (M == 2) GOLLEK_GEMM_COL_NV(T, 2);                                                              \
        else if (M == 3) GOLLEK_GEMM_COL_NV(T, 3);                                                              \
        else GOLLEK_GEMM_COL_NV(T, 4);                                                                          \
    } while (0)
    if (type_id == kQ4_K) GOLLEK_GEMM_COL(kQ4_K);
    else if (type_id == kQ5_K) GOLLEK_GEMM_COL(kQ5_K);
    else if (type_id == kQ8_0) GOLLEK_GEMM_COL(kQ8_0);
    else GOLLEK_GEMM_COL(kQ4_0);
#undef GOLLEK_GEMM_COL
#undef GOLLEK_GEMM_WIDE_NV
#undef GOLLEK_GEMM_COL_NV
    return hipGetLastError();
}

hipError_t launch_gemv_q32_mfma(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                                const float *x, float *y, int64_t rows, hipStream_t stream,
                                const uint8_t *prep, int64_t prep_rows) {
    const int nsb = (int)(cols / kQK);
    const int64_t col_rows = col_layout_rows(type_id, rows, cols);
    if (col_rows <= 0) return hipErrorInvalidValue;  // callers check q32_mfma_supported first
    const dim3 grid((unsigned)((rows + col_rows - 1) / col_rows));
    const bool use_prep = prep != nullptr && prep_rows == col_rows;
    const uint8_t *src = use_prep ? prep : w;
#define GOLLEK_COL(T)                                                                                      \
    do {                                                                                                   \
        if (nsb <= kColWaves && use_prep)                                                                  \
            hipLaunchKernelGGL((gemv_mfma_col_kernel<T, true>), grid, dim3(kColThreads), 0, stream, src,   \
                               row_bytes, nsb, x, y, rows, (int)col_rows);                                \
        else if (nsb <= kColWaves)                                                                         \
            hipLaunchKernelGGL((gemv_mfma_col_kernel<T, false>), grid, dim3(kColThreads), 0, stream, src,  \
                               row_bytes, nsb, x, y, rows, (int)col_rows);                                \
        else if (use_prep)                                                                                 \
            hipLaunchKernelGGL((gemv_mfma_wide_kernel<T, true>), grid, dim3(kColThreads), 0, stream, src,  \
                               row_bytes, nsb, x, y, rows, (int)col_rows);                                \
        else                                                                                               \
            hipLaunchKernelGGL((gemv_mfma_wide_kernel<T, false>), grid, dim3(kColThreads), 0, stream, src, \
                               row_bytes, nsb, x, y, rows, (int)col_rows);                                \
    } while (0)
    if (type_id == kQ8_0) GOLLEK_COL(kQ8_0);
    else if (type_id == kQ5_K) GOLLEK_COL(kQ5_K);
    else GOLLEK_COL(kQ4_0);
#undef GOLLEK_COL
    return hipGetLastError();
}

// Rows per workgroup of the column kernel for a full mat-vec of `rows`
// rows (0: the column kernel does not take the shape).  The prepared layout
// is laid out for this partition.
int64_t col_layout_rows(int type_id, int64_t rows, int64_t cols) {
    if (rows <= 0 || cols <= 0 || cols % kQK != 0) return 0;
    const int64_t nsb = cols / kQK, cus = device_cus();
    const int64_t per = (rows + cus - 1) / cus;
    if (nsb > 16 * kWideMaxCols) return 0;
    if (type_id == kQ4_K) {
        const int v = tuning().gemv_variant;
        if (v == 1 || v == 3) return 0;
        return per <= ColGeom<kQ4_K>::kMaxRows ? per : 0;
    }
    if (type_id != kQ4_0 && type_id != kQ8_0 && type_id != kQ5_K) return 0;
    const int v = tuning().gemv_variant;
    if (v == 1 || v == 4) return 0;
    const int64_t most = type_id == kQ8_0   ? ColGeom<kQ8_0>::kMaxRows
                         : type_id == kQ5_K ? ColGeom<kQ5_K>::kMaxRows
                                            : ColGeom<kQ4_0>::kMaxRows;
    // Q4_0 with K <= 4096: whole 16-row tiles per workgroup (4096 x 11008:
    // 48 rows on 230 workgroups, 7.0 us, against 43 on 256 with a last tile
    // of 11 rows, 7.3 us; the GGUF rows in place 7.43 against 7.47 us).
    const int64_t pp = type_id == kQ4_0 && nsb <= kColWaves ? (per + kTileRows - 1) / kTileRows * kTileRows : per;
    return pp < most ? pp : most;
}

namespace {

// Prepared layout: unit u (16 bytes) of the matrix moves from row r, byte c
// to block b = r / per (rows b per .. + nb), column c / PB, row r - b per.
__global__ void prepare_col_kernel(const uint8_t *__restrict__ raw, uint8_t *__restrict__ prep, int64_t rows,
                                   int64_t row_bytes, int64_t per, int pb) {
    const int64_t units = rows * row_bytes / 16;
    for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units;
         u += (int64_t)gridDim.x * blockDim.x) {
        const int64_t byte = 16 * u, r = byte / row_bytes, c = byte - r * row_bytes;
        const int64_t b = r / per, rr = r - b * per;
        const int64_t nb = rows - b * per < per ? rows - b * per : per;
        const int64_t col = c / pb, cc = c - col * pb;
        const int64_t dst = b * per * row_bytes + col * nb * pb + rr * pb + cc;
        *reinterpret_cast<uint4 *>(prep + dst) = *reinterpret_cast<const uint4 *>(raw + byte);
    }
}

// The inverse: GGUF rows row0 .. row0 + nrows - 1 (row_bytes each, packed
// into dst) gathered from the prepared layout.
__global__ void gather_col_rows_kernel(const uint8_t *__restrict__ prep, uint8_t *__restrict__ dst, int64_t rows,
                                       int64_t row_bytes, int64_t per, int pb, int64_t row0, int64_t nrows) {
    const int64_t units = nrows * row_bytes / 16;
    for (int64_t u = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; u < units;
         u += (int64_t)gridDim.x * blockDim.x) {
        const int64_t byte = 16 * u, rl = byte / row_bytes, c = byte - rl * row_bytes;
        const int64_t r = row0 + rl, b = r / per, rr = r - b * per;
        const int64_t nb = rows - b * per < per ? rows - b * per : per;
        const int64_t col = c / pb, cc = c - col * pb;
        const int64_t src = b * per * row_bytes + col * nb * pb + rr * pb + cc;
        *reinterpret_cast<uint4 *>(dst + byte) = *reinterpret_cast<const uint4 *>(prep + src);
    }
}

}  // namespace

// A full mat-vec from the prepared layout alone (a handle that no longer
// holds its GGUF bytes): the column / wide kernels, never a kernel that reads
// GGUF rows.  The partition must still be prep_rows and x 16-byte aligned.
hipError_t launch_gemv_prepared(int type_id, const uint8_t *prep, int64_t row_bytes, int64_t cols, const float *x,
                                float *y, int64_t rows, int64_t prep_rows, hipStream_t stream) {
    if (rows <= 0) return hipSuccess;
    if (prep == nullptr || prep_rows <= 0 || col_layout_rows(type_id, rows, cols) != prep_rows ||
        (reinterpret_cast<uintptr_t>(x) & 15u) != 0)
        return hipErrorInvalidValue;
    if (type_id == kQ4_K) return launch_gemv_q4k_mfma(prep, row_bytes, cols, x, y, rows, stream, prep, prep_rows);
    return launch_gemv_q32_mfma(type_id, prep, row_bytes, cols, x, y, rows, stream, prep, prep_rows);
}

hipError_t launch_gather_col_rows(int type_id, const uint8_t *prep, uint8_t *dst, int64_t rows, int64_t row_bytes,
                                  int64_t per, int64_t row0, int64_t nrows, hipStream_t stream) {
    if (nrows <= 0) return hipSuccess;
    const int pb = type_id == kQ8_0 ? ColGeom<kQ8_0>::PB : type_id == kQ5_K ? ColGeom<kQ5_K>::PB : ColGeom<kQ4_K>::PB;
    const int64_t units = nrows * row_bytes / 16;
    const int64_t blocks = (units + 255) / 256 < 65536 ? (units + 255) / 256 : 65536;
    hipLaunchKernelGGL(gather_col_rows_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, prep, dst, rows,
                       row_bytes, per, pb, row0, nrows);
    return hipGetLastError();
}

// The column kernel's prepared layout of a full matrix (rows x row_bytes)
// for col_layout_rows(...) = per rows per workgroup; every piece is a whole
// number of 16-byte units, so units move whole.
hipError_t launch_prepare_col_layout(int type_id, const uint8_t *raw, uint8_t *prep, int64_t rows,
                                     int64_t row_bytes, int64_t per, hipStream_t stream) {
    const int pb = type_id == kQ8_0 ? ColGeom<kQ8_0>::PB : type_id == kQ5_K ? ColGeom<kQ5_K>::PB : ColGeom<kQ4_K>::PB;
    const int64_t units = rows * row_bytes / 16;
    const int64_t blocks = (units + 255) / 256 < 65536 ? (units + 255) / 256 : 65536;
    hipLaunchKernelGGL(prepare_col_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, raw, prep, rows, row_bytes,
                       per, pb);
    return hipGetLastError();
}

}  // namespace gollek
