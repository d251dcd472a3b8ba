// gguf_gemv_ring.hip -- Q8_0 / Q4_0 fused dequant-GEMV (M = 1) streaming the
// weights through per-wave buffer->LDS rings.
//
// y[r] = sum_b d_b * sum_i q_{b,i} x_{32 b + i}, the raw routes of
// RT/GgufQ8RawDot.java:137-184 (Q8_0) and RT/GgufQ40RawDot.java (Q4_0, q =
// nibble - 8; RT/ = runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/
// gollek/gguf/runtime/), in fp32.
//
// A workgroup of W waves (4..16, chosen so that large matrices get about
// one workgroup per CU and stage x once per CU) owns 4 W consecutive rows;
// wave w owns rows 4w .. 4w + 3 and streams them in items of 16 blocks (544 bytes of each row
// for Q8_0, 288 for Q4_0) through a ring of NS slots of its own, so the waves
// never wait for each other: each row's item piece is contiguous in memory
// and lands as 16-byte chunks (4 rows x 34 or 18 chunks: three or two load
// instructions, the last one partly masked).  x (fp32) is staged once per
// workgroup in LDS.  Lane
// (row r = lane / 16, block b = lane % 16) contracts its block's 32 quants
// in order with fp32 FMAs (int8 bytes widen with one sign-extending SDWA
// convert each; Q4_0 nibbles with an unsigned convert and an exact - 8) and
// adds d_b times that sum to its partial, the block
// structure of the reference; the 16 lanes of a row meet in a shuffle
// reduction at the end.  x sits in LDS at 144 bytes per 32-float block (16
// bytes of padding), so the 16 lanes' 16-byte reads of 16 blocks fall in
// distinct banks.  All LDS reads of bytes written by
// buffer->LDS loads are inline asm: the compiler cannot tell which load
// wrote which bytes and would otherwise wait for every load in flight.
#include <type_traits>

#include "gguf_blocks.hpp"
#include "gguf_dot4.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

namespace {

constexpr int kGrWaveRows = 4;   // rows per wave
constexpr int kGrMaxWaves = 16;  // waves per workgroup
constexpr int kGrIB = 16;        // blocks per item
constexpr int kGrMaxK = 16384;   // x floats held in LDS

template <int TYPE>
struct GrFmt;
template <>
struct GrFmt<kQ8_0> {
    static constexpr int kBlockBytes = kQ8BlockBytes;  // 34: d, 32 int8 quants
    static constexpr int kQDwords = 9;                 // dwords covering a block's quants
};
template <>
struct GrFmt<kQ4_0> {
    static constexpr int kBlockBytes = kQ4BlockBytes;  // 18: d, 16 bytes of nibbles
    static constexpr int kQDwords = 5;
};
template <int TYPE>
struct GrItem {
    static constexpr int kPiece = kGrIB * GrFmt<TYPE>::kBlockBytes;  // bytes of a row per item
    static constexpr int kChunks = kPiece / 16;                      // 16-byte chunks of a row
    static constexpr int kDma = (4 * kChunks + 63) / 64;             // loads per item and wave
    static constexpr int kSlot = 1024 * kDma;                        // masked lanes land in the pad
};

// Dynamic LDS: x (144 bytes per 32-float block), then the waves' rings.
constexpr int kGrXBlock = 144;
__host__ __device__ constexpr int gr_x_bytes(int K) { return K / 32 * kGrXBlock; }
__host__ __device__ constexpr int gr_ring_offset(int K) { return gr_x_bytes(K); }
template <int TYPE>
__host__ __device__ constexpr int gr_lds_bytes(int K, int NS, int waves) {
    return gr_ring_offset(K) + waves * NS * GrItem<TYPE>::kSlot;
}

extern __shared__ __attribute__((aligned(16))) uint8_t gr_dyn_lds[];

template <bool NT>
__device__ __forceinline__ void gr_dma16(__amdgpu_buffer_rsrc_t rs, uint8_t *dst, uint32_t off) {
    if constexpr (NT)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)dst, 16, off, 0, 0, kStreamLoad);
    else
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)dst, 16, off, 0, 0, 0);
}

template <int N>
__device__ __forceinline__ void gr_wait_vm() {
    asm volatile("s_waitcnt vmcnt(%0)" : : "n"(N) : "memory");
}

// ND raw dwords from `a` (a block's quants, realigned by the caller) and
// the scale dword `as`.
template <int ND>
__device__ __forceinline__ void gr_read_w(uint32_t a, uint32_t as, uint32_t (&q)[ND], uint32_t &sc) {
    uint2 p0, p1, p2, p3;
    if constexpr (ND == 5) {
        asm volatile(
            "ds_read2_b32 %0, %4 offset0:0 offset1:1\n\t"
            "ds_read2_b32 %1, %4 offset0:2 offset1:3\n\t"
            "ds_read_b32 %2, %4 offset:16\n\t"
            "ds_read_b32 %3, %5\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(p0), "=&v"(p1), "=&v"(q[4]), "=&v"(sc)
            : "v"(a), "v"(as)
            : "memory");
    } else {
        asm volatile(
            "ds_read2_b32 %0, %6 offset0:0 offset1:1\n\t"
            "ds_read2_b32 %1, %6 offset0:2 offset1:3\n\t"
            "ds_read2_b32 %2, %6 offset0:4 offset1:5\n\t"
            "ds_read2_b32 %3, %6 offset0:6 offset1:7\n\t"
            "ds_read_b32 %4, %6 offset:32\n\t"
            "ds_read_b32 %5, %7\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(p0), "=&v"(p1), "=&v"(p2), "=&v"(p3), "=&v"(q[ND - 1]), "=&v"(sc)
            : "v"(a), "v"(as)
            : "memory");
        q[4] = p2.x;
        q[5] = p2.y;
        q[6] = p3.x;
        q[7] = p3.y;
    }
    q[0] = p0.x;
    q[1] = p0.y;
    q[2] = p1.x;
    q[3] = p1.y;
}

// N consecutive floats of x (N / 4 reads of 16 bytes).
template <int N>
__device__ __forceinline__ void gr_read_x(uint32_t a, float (&x)[N]) {
    u32x4 v[N / 4];
    if constexpr (N == 16) {
        asm volatile(
            "ds_read_b128 %0, %4\n\t"
            "ds_read_b128 %1, %4 offset:16\n\t"
            "ds_read_b128 %2, %4 offset:32\n\t"
            "ds_read_b128 %3, %4 offset:48\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3])
            : "v"(a)
            : "memory");
    } else {
        asm volatile(
            "ds_read_b128 %0, %8\n\t"
            "ds_read_b128 %1, %8 offset:16\n\t"
            "ds_read_b128 %2, %8 offset:32\n\t"
            "ds_read_b128 %3, %8 offset:48\n\t"
            "ds_read_b128 %4, %8 offset:64\n\t"
            "ds_read_b128 %5, %8 offset:80\n\t"
            "ds_read_b128 %6, %8 offset:96\n\t"
            "ds_read_b128 %7, %8 offset:112\n\t"
            "s_waitcnt lgkmcnt(0)"
            : "=&v"(v[0]), "=&v"(v[1]), "=&v"(v[2]), "=&v"(v[3]), "=&v"(v[4]), "=&v"(v[5]),
              "=&v"(v[6]), "=&v"(v[7])
            : "v"(a)
            : "memory");
    }
#pragma unroll
    for (int i = 0; i < N / 4; i++) {
        x[4 * i + 0] = __uint_as_float(v[i].x);
        x[4 * i + 1] = __uint_as_float(v[i].y);
        x[4 * i + 2] = __uint_as_float(v[i].z);
        x[4 * i + 3] = __uint_as_float(v[i].w);
    }
}

// Sign-extended byte k of w as a float (one SDWA convert).
__device__ __forceinline__ float gr_sbyte(uint32_t w, int k) {
    return (float)(int)(int8_t)(uint8_t)(w >> (8 * k));
}

}  // namespace

template <int TYPE, int NS, bool NT>
__global__ __launch_bounds__(64 * kGrMaxWaves) void gemv_ring_kernel(const uint8_t *__restrict__ w,
                                                        int64_t row_bytes, int K,
                                                        const float *__restrict__ x,
                                                        float *__restrict__ y, int64_t rows) {
    using F = GrFmt<TYPE>;
    using I = GrItem<TYPE>;
    constexpr int IB = kGrIB;
    constexpr int PIECE = I::kPiece;  // 544 / 288 bytes of a row per item
    constexpr int CH = I::kChunks;    // 34 / 18 chunks
    constexpr int DMA = I::kDma;      // 3 / 2 loads
    constexpr int ND = F::kQDwords;
    static_assert(PIECE % 16 == 0, "item layout");
    uint8_t *const lds = gr_dyn_lds;
    const int tid = threadIdx.x;
    const int nt = (int)blockDim.x;  // 64 x waves
    const int lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int64_t row0 = (int64_t)blockIdx.x * (kGrWaveRows * (nt >> 6));
    // K a multiple of 32: the last item may hold fewer than IB blocks; its
    // lanes past the row's last block read bytes of the next row (or zeros
    // past the wave's rows) and x past K (LDS of the ring), and add nothing.
    const int nblocks = K / 32;
    const int nitems = (nblocks + IB - 1) / IB;

    uint8_t *const xl = lds;
    uint8_t *const ring = lds + gr_ring_offset(K) + wave * NS * I::kSlot;

    // The wave's four rows (zeros past `rows`).  Loads of items past the last
    // one read the following bytes of the buffer (or zeros past its end)
    // into slots that are never used.
    const int64_t r_first = row0 + 4 * wave;
    const int64_t nr = rows - r_first < 4 ? (rows - r_first > 0 ? rows - r_first : 0) : 4;
    const __amdgpu_buffer_rsrc_t ws =
        wave_buffer(w + (nr > 0 ? r_first : 0) * row_bytes, (uint32_t)(nr * row_bytes));
    // Chunk c = 64 i + lane of an item: row c / CH, part c % CH.
    uint32_t wo[DMA];
#pragma unroll
    for (int i = 0; i < DMA; i++) {
        const int c = 64 * i + lane;
        wo[i] = c < 4 * CH ? (uint32_t)(c / CH) * (uint32_t)row_bytes + 16u * (uint32_t)(c % CH)
                           : kMaskedOffset;
    }
    auto issue = [&](int j, uint8_t *slot) {
        const uint32_t jo = (uint32_t)j * (uint32_t)PIECE;
#pragma unroll
        for (int i = 0; i < DMA; i++)
            gr_dma16<NT>(ws, slot + 1024 * i, wo[i] == kMaskedOffset ? kMaskedOffset : wo[i] + jo);
    };

    // x: thread t takes floats 16 t' .. 16 t' + 15 for t' = t, t + nt, ...
    // (at most four, as K <= 16384 and nt >= 256)
    // (half of block t' / 2), loaded to registers before the ring prologue
    // and written to the padded layout after it.
    const __amdgpu_buffer_rsrc_t xrs = wave_buffer(reinterpret_cast<const uint8_t *>(x), (uint32_t)(4 * K));
    const int xparts = K / 16;
    u32x4 xr[4][4];
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int tp = tid + nt * u;
#pragma unroll
        for (int i = 0; i < 4; i++)
            xr[u][i] = __builtin_amdgcn_raw_buffer_load_b128(xrs, tp < xparts ? (uint32_t)(64 * tp + 16 * i) : kMaskedOffset, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);  // every x load ahead of the ring loads
#pragma unroll
    for (int j = 0; j < NS - 1; j++) issue(j, ring + j * I::kSlot);
    const uint32_t xl_base = (uint32_t)(uintptr_t)(lds_ptr)xl;
#pragma unroll
    for (int u = 0; u < 4; u++) {
        const int tp = tid + nt * u;
        if (tp < xparts) {
            const uint32_t a = xl_base + (uint32_t)(kGrXBlock * (tp >> 1) + 64 * (tp & 1));
            asm volatile(
                "ds_write_b128 %0, %1\n\t"
                "ds_write_b128 %0, %2 offset:16\n\t"
                "ds_write_b128 %0, %3 offset:32\n\t"
                "ds_write_b128 %0, %4 offset:48"
                :
                : "v"(a), "v"(xr[u][0]), "v"(xr[u][1]), "v"(xr[u][2]), "v"(xr[u][3])
                : "memory");
        }
    }
    // Consume every x register on every path: a load whose result is left
    // unused on some path makes the compiler wait for all loads (the ring's
    // included) where the paths meet.
#pragma unroll
    for (int u = 0; u < 4; u++)
        asm volatile("" : : "v"(xr[u][0]), "v"(xr[u][1]), "v"(xr[u][2]), "v"(xr[u][3]));
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");

    // Lane roles: row r = lane / 16, block b = lane % 16 of the item.  Q4_0
    // quants: low nibbles are quants 0..15, high nibbles 16..31.
    const int r = lane >> 4;
    const int b = lane & 15;
    const int qoff = r * PIECE + b * F::kBlockBytes + 2;  // first quant byte in the slot
    const uint32_t q_rel = (uint32_t)(qoff & ~3);
    const uint32_t q_sh = (uint32_t)(qoff & 3);                   // 0 or 2
    const int soff = r * PIECE + b * F::kBlockBytes;              // scale bytes
    const uint32_t s_rel = (uint32_t)(soff & ~3);
    const uint32_t s_sh = (uint32_t)(8 * (soff & 3));             // 0 or 16
    const uint32_t ring_base = (uint32_t)(uintptr_t)(lds_ptr)ring;
    const uint32_t x_lane = xl_base + (uint32_t)(kGrXBlock * b);

    float acc = 0.0f;
    int sl = 0;
    for (int j = 0; j < nitems; j++) {
        gr_wait_vm<DMA * (NS - 2)>();  // item j has landed
        issue(j + NS - 1, ring + (sl == 0 ? NS - 1 : sl - 1) * I::kSlot);
        const uint32_t sb = ring_base + (uint32_t)(sl * I::kSlot);
        uint32_t q[ND], sc;
        gr_read_w<ND>(sb + q_rel, sb + s_rel, q, sc);
        uint32_t qa[ND - 1];
#pragma unroll
        for (int i = 0; i < ND - 1; i++) qa[i] = __builtin_amdgcn_alignbyte(q[i + 1], q[i], q_sh);
        const float d = half_bits_to_float_fast((sc >> s_sh) & 0xFFFFu);
        if constexpr (TYPE == kQ8_0) {
            float xv[32];
            gr_read_x<32>(x_lane + (uint32_t)(kGrXBlock * IB * j), xv);
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 32; i++) s = fmaf(gr_sbyte(qa[i >> 2], i & 3), xv[i], s);
            acc = IB * j + b < nblocks ? fmaf(d, s, acc) : acc;
        } else {
            // (q - 8) x per element, as the reference does: the offset is
            // exact in fp32 and nothing cancels.
            float xv[32];
            gr_read_x<32>(x_lane + (uint32_t)(kGrXBlock * IB * j), xv);
            float s = 0.0f;
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const uint32_t lo = opaque(qa[i] & 0x0F0F0F0Fu);
                const uint32_t hi = opaque((qa[i] >> 4) & 0x0F0F0F0Fu);
#pragma unroll
                for (int k = 0; k < 4; k++) {
                    s = fmaf(byte_f(lo, k) - 8.0f, xv[4 * i + k], s);
                    s = fmaf(byte_f(hi, k) - 8.0f, xv[16 + 4 * i + k], s);
                }
            }
            acc = IB * j + b < nblocks ? fmaf(d, s, acc) : acc;
        }
        sl = sl + 1 == NS ? 0 : sl + 1;
    }
    gr_wait_vm<0>();  // the loads issued past the last item
    // Sum the 16 lanes of each row.
#pragma unroll
    for (int m = 8; m >= 1; m >>= 1) acc += __shfl_xor(acc, m, 64);
    const int64_t row = r_first + r;
    if ((lane & 15) == 0 && r < nr) y[row] = acc;
}

namespace {

template <int TYPE, int NS, bool NT = true>
hipError_t launch_ring(const uint8_t *w, int64_t row_bytes, int64_t cols, const float *x, float *y,
                       int64_t rows, hipStream_t stream) {
    // Waves per workgroup: enough rows that the grid is about one workgroup
    // per CU (each workgroup stages all of x), at least four, within LDS.
    const int64_t cus = device_cus();
    const int lds_cap = 160 * 1024;
    int waves = (int)((rows + kGrWaveRows * cus - 1) / (kGrWaveRows * cus));
    if (waves < 4) waves = 4;
    if (waves > kGrMaxWaves) waves = kGrMaxWaves;
    while (waves > 4 && gr_lds_bytes<TYPE>((int)cols, NS, waves) > lds_cap) waves--;
    const int64_t wg_rows = (int64_t)kGrWaveRows * waves;
    const unsigned grid = (unsigned)((rows + wg_rows - 1) / wg_rows);
    const int lds = gr_lds_bytes<TYPE>((int)cols, NS, waves);
    if (lds > 65536) {
        const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(&gemv_ring_kernel<TYPE, NS, NT>),
                                                 hipFuncAttributeMaxDynamicSharedMemorySize, lds);
        if (e != hipSuccess) return e;
    }
    hipLaunchKernelGGL((gemv_ring_kernel<TYPE, NS, NT>), dim3(grid), dim3(64 * waves), (size_t)lds, stream, w,
                       row_bytes, (int)cols, x, y, rows);
    return hipGetLastError();
}

}  // namespace

bool gemv_ring_supported(int type_id, int64_t row_bytes, int64_t cols, int64_t rows, const void *w,
                         const float *x) {
    if (type_id != kQ8_0 && type_id != kQ4_0) return false;
    if (tuning().gemv_variant == 1) return false;
    const int bb = type_id == kQ8_0 ? kQ8BlockBytes : kQ4BlockBytes;
    return cols > 0 && cols % 32 == 0 && cols <= kGrMaxK && row_bytes == cols / 32 * bb &&
           (row_bytes & 3) == 0 && (reinterpret_cast<uintptr_t>(w) & 3u) == 0 &&
           (reinterpret_cast<uintptr_t>(x) & 3u) == 0 && 4 * row_bytes < ((int64_t)1 << 31) &&
           rows > 0;
}

hipError_t launch_gemv_ring(int type_id, const uint8_t *w, int64_t row_bytes, int64_t cols,
                            const float *x, float *y, int64_t rows, hipStream_t stream) {
    // Measured on MI355X (Q8_0 4096 x 4096, Q4_0 11008 x 4096): three slots
    // per wave beat deeper rings, which only queue more requests at the HBM;
    // the streaming cache policy makes no difference.
    if (type_id == kQ8_0) return launch_ring<kQ8_0, 3>(w, row_bytes, cols, x, y, rows, stream);
    return launch_ring<kQ4_0, 3>(w, row_bytes, cols, x, y, rows, stream);
}

}  // namespace gollek
