// gguf_moe_mfma.hip -- grouped MoE expert FFN on the gfx950 matrix cores:
// Q4_K, Q5_K or Q6_K gate / up experts (Q6_K up to hidden 2048) with Q4_K,
// Q5_K or Q6_K down experts, and all-Q4_0 experts.
//
// Semantics as gguf_moe.hip (MoeForwardPass.java:217-240, :461-472; swigluFfn
// DirectForwardFfnService.java:40-61): h_pair = silu(gate_e x_t) * (up_e x_t),
// y_pair = down_e h_pair, out[t] = sum_j w[t,j] y_pair[t,j] in route order.
//
// Two passes of one tile kernel.  Each workgroup first sorts the valid
// routes by expert and lays out the work items itself, in LDS (routing is a
// few microseconds of latency as a launch of its own, and tables in global
// memory would put dependent reads in front of the first weight load):
//   pass 0 (gate/up): item = (used expert, 16-row tile of its I rows, group of
//     up to 4 of its routes).  A slot holds the tile's 16 gate rows and 16 up
//     rows; wave w < nsb contracts gate superblock w, wave nsb + w up
//     superblock w; h = silu(g) u per route and row.
//   pass 1 (down): item = (used expert, RT (at most 16 / nsb, as a slot
//     holds) 16-row tiles of its H rows, route group); wave w = (row tile
//     w / nsb, superblock w % nsb).  With inter sizes up to 1024 and Q4_K,
//     Q5_K or Q6_K down rows, pass 0 leaves h as digit records and the
//     token-major moe_down_combine_kernel replaces pass 1 and the combine.
// The K-quant contraction is the one of gguf_gemv_mfma.hip's kernels
// (v_mfma_i32_16x16x64_i8 over balanced 22-bit digits of the vector, low and
// high nibbles as bytes 0..15, Q5_K's fifth bits from qh added as bit 4),
// with two routes per MFMA: A rows 8 t + 4 h + p hold route t's digits, so its
// results sit in output lanes 32 t + 16 h + n and the second route costs no
// extra epilogue instructions.  Q4_0 rows are read as 144-byte pieces of
// eight blocks.
//
// Every used expert's weights stream from HBM once per group of four routes
// (routing spreads 16 tokens x top-8 over 128 experts at ~1 route per
// expert).  When the (expert, route group) units fit the grid, each unit
// gets its own workgroups, each an even slice of it; otherwise the
// workgroups split the flattened item list evenly.  A wave builds its digit
// operands from the float vectors (x for pass 0, h for pass 1) at the start
// and whenever the route group changes, which drains the load pipeline
// once.  Results collect in LDS and are stored at those drains, when the
// buffer fills and at the end: on gfx9 stores share the load counter the
// ring waits on.  Items stream through a ring of slots in LDS (MoRing):
// three of 38 KB, or for Q5_K rows two of 46 KB.
#include <type_traits>

#include "gguf_dot4.hpp"
#include "gguf_kernels.hpp"
#include "gguf_mfma_q4k.hpp"

namespace gollek {

using namespace mfq;

namespace {

constexpr int kMoWaves = 16;
constexpr int kMoThreads = kMoWaves * 64;
constexpr int kMoGroup = 4;          // routes per group (two MFMA pairs)
// The item ring: three slots of 38 KB; for Q5_K rows (176-byte
// superblocks) two slots of 46 KB and for Q6_K rows (210 bytes) two of 54
// KB, so that 16 gate and 16 up rows of 8 superblocks (hidden 2048) fit one
// slot.
template <int WT>
struct MoRing {
    static constexpr int kMaxDma = WT == kQ6_K ? 54 : WT == kQ5_K ? 46 : 38;  // 1 KB loads per item slot
    static constexpr int kSlots = WT == kQ5_K || WT == kQ6_K ? 2 : 3;
    static constexpr int kSlot = kMaxDma * 1024;
    static constexpr int kDmaPerWave = (kMaxDma + kMoWaves - 1) / kMoWaves;
};
constexpr int kMoOutCap = 1536;      // buffered results (value, index)
constexpr int kMoMaxExperts = 256;   // routing tables held in LDS
constexpr int kMoMaxRoutes = kMoeMfmaMaxRoutes;

// Routing tables of one pass, built in LDS by every workgroup: the valid
// routes (expert id in range, weight != 0; MoeForwardPass.java:222) stably
// sorted by expert (pairs), each expert's first slot in that order
// (offsets[e], offsets[E] = valid routes), the used experts in expert order
// and per used expert u the first work item items[u] (items[nused] = all).
struct MoeRouteLds {
    int32_t offsets[kMoMaxExperts + 1];
    int32_t used[kMoMaxExperts];
    int32_t items[kMoMaxExperts + 1];
    int32_t nused;
    uint16_t pairs[kMoMaxRoutes];
};

// Inclusive prefix sum over the wave (DPP: shifts within rows of 16, then
// the row totals broadcast to the rows above).
__device__ __forceinline__ int wave_scan_incl(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xF, 0xF, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xF, 0xF, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xF, 0xF, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xF, 0xF, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xA, 0xF, false);  // row_bcast:15 -> rows 1, 3
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xC, 0xF, false);  // row_bcast:31 -> rows 2, 3
    return v;
}

// Builds R for work units of tiles_e items per (expert, group of `group`
// routes).  tmp: P + E ints of LDS that nothing else uses meanwhile.  Every
// thread of the workgroup calls this; it ends with a barrier.  Counts by LDS
// atomics, then wave 0 scans the experts in chunks of 64 (wave_scan_incl)
// and scatters the routes 64 at a time in route order: a route's slot is its
// expert's running offset plus its rank among the chunk's equal keys (found
// by ballots over the key bits).
__device__ void moe_route_lds(const int32_t *__restrict__ ids, const float *__restrict__ wts, int P,
                              int E, int tiles_e, int group, MoeRouteLds &R, int32_t *tmp) {
    int32_t *keys = tmp, *run = tmp + P;
    const int tid = (int)threadIdx.x, lane = tid & 63;
    for (int e = tid; e < E; e += (int)blockDim.x) run[e] = 0;
    __syncthreads();
    for (int p = tid; p < P; p += (int)blockDim.x) {
        const int e = ids[p];
        const bool valid = e >= 0 && e < E && wts[p] != 0.0f;
        if (valid) atomicAdd(&run[e], 1);  // LDS atomic
        keys[p] = valid ? e : -1;
    }
    __syncthreads();
    if (tid < 64) {
        const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        int carry = 0, ucount = 0, icarry = 0;
        for (int base = 0; base < E; base += 64) {
            const int e = base + lane;
            const int c = e < E ? run[e] : 0;
            const int units = tiles_e * ((c + group - 1) / group);
            const int a = wave_scan_incl(c), b = wave_scan_incl(units);
            const uint64_t ub = __ballot(c > 0);
            if (e < E) {
                R.offsets[e] = carry + a - c;
                run[e] = carry + a - c;
            }
            if (c > 0) {
                const int u = ucount + __popcll(ub & below);
                R.used[u] = e;
                R.items[u] = icarry + b - units;
            }
            carry += __builtin_amdgcn_readlane(a, 63);
            icarry += __builtin_amdgcn_readlane(b, 63);
            ucount += __popcll(ub);
        }
        if (lane == 0) {
            R.offsets[E] = carry;
            R.nused = ucount;
            R.items[ucount] = icarry;
        }
        int bits = 1;
        while ((1 << bits) <= E) bits++;
        for (int base = 0; base < P; base += 64) {
            const int p = base + lane;
            const int key = p < P ? keys[p] : -1;
            const uint32_t k1 = (uint32_t)(key + 1);
            uint64_t same = __ballot(true);
            for (int bt = 0; bt < bits; bt++) {
                const uint64_t v = __ballot((k1 >> bt) & 1u);
                same &= ((k1 >> bt) & 1u) ? v : ~v;
            }
            const int rank = __popcll(same & below);
            const int r0 = key >= 0 ? run[key] : 0;  // read by all lanes before any update
            if (key >= 0) R.pairs[r0 + rank] = (uint16_t)p;
            const bool last = (same >> lane) == 1ull;  // highest lane of its key
            if (key >= 0 && last) run[key] = r0 + __popcll(same);
        }
    }
    __syncthreads();
}

}  // namespace

// Host-computed geometry of one pass.
struct MoeTileGeom {
    int nsb;          // superblocks per item row (K / 256, over halves)
    int halves;       // K-halves per tile (pass 0 with K > 2048: 2; else 1)
    int rows_e;       // weight rows per expert
    int rt;           // 16-row tiles per item (pass 0: 1)
    int tiles_e;      // items per expert and route group (tiles x halves)
    uint32_t row_bytes, pitch;  // bytes of an item's row, its LDS pitch
    uint32_t stride;  // bytes of a weight row (halves x row_bytes)
    int part_dma;     // loads per matrix part (pass 0) or per item (pass 1)
    int ndma;         // loads per item
    int vec_len;      // vector length (K)
    int out_len;      // result length per route (rows per expert)
    int64_t w_bytes;  // bytes of one stacked weight matrix (< 2^31)
};

// One route's 16 h values as a digit record (every lane of the wave calls
// this; lanes 16 k .. 16 k + 15 hold one route's elements r = lane & 15):
// three balanced signed-byte planes of the integers
// X_r = rint(h_r / 2^(e-22)), max |h| < 2^e over the 16, so |X_r| <= 2^22
// and an element's error is at most 2^-23 of that maximum; plane-major:
// lane r returns dword 4 (r & 3) + (r >> 2) = plane r & 3 of elements
// 4 (r >> 2) .. + 3 (plane 3 is zero and not stored); `scale` = 2^(e-22)
// (NaN when an h is not finite) and `sum` = the fp32 sum of the 16 h, in
// every lane.
__device__ __forceinline__ uint32_t h_record16(float hval, float &scale, float &sum) {
    uint32_t mb = __float_as_uint(hval) & 0x7FFFFFFFu;
    mb = max(mb, (uint32_t)dpp_i<0xB1>((int)mb));   // quad_perm [1,0,3,2]
    mb = max(mb, (uint32_t)dpp_i<0x4E>((int)mb));   // quad_perm [2,3,0,1]
    mb = max(mb, (uint32_t)dpp_i<0x124>((int)mb));  // row_ror:4
    mb = max(mb, (uint32_t)dpp_i<0x128>((int)mb));  // row_ror:8
    const bool finite = mb < 0x7F800000u;
    int e = 0;
    (void)frexpf(__uint_as_float(mb), &e);
    const int X = finite ? (int)rintf(ldexpf(hval, 22 - e)) : 0;  // |X| <= 2^22
    // Adding 0x8080 makes bytes 0, 1 the digits + 128; the XOR maps them back
    // to signed bytes and leaves the top digit (X + 0x8080) >> 16 in
    // [-64, 64] as byte 2.
    const uint32_t Y = ((uint32_t)X + 0x00008080u) ^ 0x00008080u;
    float s = hval;
    s += __int_as_float(dpp_i<0xB1>(__float_as_int(s)));
    s += __int_as_float(dpp_i<0x4E>(__float_as_int(s)));
    s += __int_as_float(dpp_i<0x124>(__float_as_int(s)));
    s += __int_as_float(dpp_i<0x128>(__float_as_int(s)));
    sum = s;
    scale = finite ? ldexpf(1.0f, e - 22) : __builtin_nanf("");
    // lane 4 j + p: byte p of the quad's four Y (quad_perm broadcasts)
    const uint32_t y0 = (uint32_t)dpp_i<0x00>((int)Y), y1 = (uint32_t)dpp_i<0x55>((int)Y);
    const uint32_t y2 = (uint32_t)dpp_i<0xAA>((int)Y), y3 = (uint32_t)dpp_i<0xFF>((int)Y);
    const uint32_t pb = (uint32_t)(threadIdx.x & 3);
    const uint32_t sel = pb | ((pb + 4u) << 8) | 0x0C0C0000u;
    return __builtin_amdgcn_perm(y1, y0, sel) | (__builtin_amdgcn_perm(y3, y2, sel) << 16);
}

// h record of route p and 16-element group G (groups = I / 16 per route):
// 14 dwords at 14 (p groups + G): the 12 plane dwords of h_record16, then
// scale and sum, so one route's records are one contiguous run.
constexpr int kRecDwords = 14;

// MODE 0: gate/up (w0 = gate, w1 = up); MODE 1: down (w0 = down).
// REC (MODE 0): h leaves as records (kRecDwords) for moe_down_combine_kernel;
// otherwise as fp32 (out + p I + row).
// vec: pass 0 x[T][H] (route p -> token p / top_k); pass 1 h[P][I] (route p).
// HV (MODE 0): K-halves per tile.  With HV = 2 (hidden sizes past 2048) a
// tile's two halves are consecutive items, each wave keeps both halves' x
// operands, and the first half's gate / up row sums wait in LDS (hsave)
// for the second's, so h = silu(gate) * up is formed once per row.
template <int MODE, bool REC, int HV = 1, int WT = kQ4_K>
__global__ __launch_bounds__(kMoThreads) void moe_expert_tile_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, MoeTileGeom G,
    const float *__restrict__ vec, int top_k, const int32_t *__restrict__ ids,
    const float *__restrict__ wts, int E, int P, float *__restrict__ out) {
    static_assert(MODE == 0 || !REC, "records are pass 0's output");
    static_assert(HV == 1 || (HV == 2 && MODE == 0), "K-halves in pass 0 only");
    static_assert(WT == kQ4_K || WT == kQ5_K || (WT == kQ4_0 && HV == 1) || (WT == kQ6_K && HV == 1 && MODE == 0),
                  "Q4_0 rows in one half; Q6_K gate / up rows in one half");
    // bytes of a 256-column piece of a row (eight Q4_0 blocks are 144, as a
    // Q4_K superblock)
    constexpr uint32_t PB = WT == kQ6_K ? 210u : WT == kQ5_K ? kQ5KBlockBytes : kQKBlockBytes;
    // routes per group: Q6_K takes one route per MFMA (its 16-element scale
    // groups need 12 A rows), so two routes' operands fill the registers
    // four take for the other types
    constexpr int kGrp = WT == kQ6_K ? 2 : kMoGroup;
    using RG = MoRing<WT>;
    constexpr int kMoMaxDma = RG::kMaxDma, kMoSlots = RG::kSlots, kMoSlot = RG::kSlot;
    constexpr int kMoDmaPerWave = RG::kDmaPerWave;
    __shared__ __attribute__((aligned(16))) uint8_t ring[kMoSlots * kMoSlot + 1024];  // + sink
    // digit build; HV = 2: + the (half, route) x sums and scales from 768
    __shared__ __attribute__((aligned(16))) uint8_t scratch[kMoWaves][HV == 2 ? 1088 : 1024];
    __shared__ float part[2][kMoGroup][kMoWaves][16];
    __shared__ float outv[kMoOutCap];
    __shared__ int outi[kMoOutCap];
    __shared__ int gid[kMoGroup];  // route ids of the current group
    __shared__ float hsave[HV == 2 ? kMoGroup * 16 : 1][2];  // first-half gate / up sums
    __shared__ MoeRouteLds R;

    // Routing (the ring is free until the first loads below).
    moe_route_lds(ids, wts, P, E, G.tiles_e, kGrp, R, reinterpret_cast<int32_t *>(ring));
    const int32_t *offsets = R.offsets, *used = R.used, *items = R.items;
    const uint16_t *pairs = R.pairs;
    const int nused = R.nused;
    const int nitems = items[nused];
    // Work split.  Every (expert, route group) unit has G.tiles_e items, in
    // order.  When k = grid / units workgroups per unit leave at most 1/8 of
    // the grid idle, unit j gets workgroups k j .. k j + k - 1 and each takes
    // an even slice of it, so no workgroup changes route group (which costs a
    // pipeline drain); otherwise the items are split evenly over the grid.
    const int nunits = nitems / G.tiles_e;
    const int kpu = nunits > 0 ? (int)gridDim.x / nunits : 0;
    const bool unit_split = kpu >= 1 && 8 * ((int)gridDim.x - kpu * nunits) <= (int)gridDim.x;
    int i_begin, i_end;
    // Slices are whole tiles (HV items each), so a tile's halves stay in
    // one workgroup.
    const int tpu = G.tiles_e / HV, ntiles = nitems / HV;
    if (unit_split) {
        const int unit = (int)blockIdx.x / kpu, sub = (int)blockIdx.x - unit * kpu;
        i_begin = unit < nunits ? unit * G.tiles_e + HV * (sub * tpu / kpu) : 0;
        i_end = unit < nunits ? unit * G.tiles_e + HV * ((sub + 1) * tpu / kpu) : 0;
    } else {
        i_begin = HV * (int)((int64_t)blockIdx.x * ntiles / gridDim.x);
        i_end = HV * (int)((int64_t)(blockIdx.x + 1) * ntiles / gridDim.x);
    }
    if (i_begin >= i_end) return;  // uniform, before any barrier

    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int rows_item = 16 * G.rt;
    const __amdgpu_buffer_rsrc_t rs0 = wave_buffer(w0, (uint32_t)G.w_bytes);
    const __amdgpu_buffer_rsrc_t rs1 = wave_buffer(MODE == 0 ? w1 : w0, (uint32_t)G.w_bytes);

    // Items in order (wave-uniform): a cursor steps tile, then route group,
    // then used expert, and reads the routing tables only when it moves to
    // the next expert (dependent table reads per item would sit on the
    // critical path after every barrier).
    struct Item {
        int u, e, group, tile, half, ntok, row0, nrows;
    };
    struct Cursor {
        int u, e, cnt, groups, group, tile;
    };
    auto cursor_at = [&](int i) {
        Cursor c;
        int lo = 0, hi = nused - 1;  // last u with items[u] <= i (binary search)
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (items[mid] <= i) lo = mid;
            else hi = mid - 1;
        }
        c.u = lo;
        c.e = used[c.u];
        c.cnt = offsets[c.e + 1] - offsets[c.e];
        c.groups = (c.cnt + kGrp - 1) / kGrp;
        const int j = i - items[c.u];
        c.group = j / G.tiles_e;
        c.tile = j - c.group * G.tiles_e;
        return c;
    };
    auto step = [&](Cursor &c) {
        if (++c.tile < G.tiles_e) return;
        c.tile = 0;
        if (++c.group < c.groups) return;
        c.group = 0;
        if (++c.u < nused) {
            c.e = used[c.u];
            c.cnt = offsets[c.e + 1] - offsets[c.e];
            c.groups = (c.cnt + kGrp - 1) / kGrp;
        }
    };
    auto item_of = [&](const Cursor &c) {
        Item it;
        it.u = c.u;
        it.e = c.e;
        it.group = c.group;
        it.tile = c.tile / HV;
        it.half = c.tile - HV * it.tile;
        it.ntok = min(kGrp, c.cnt - kGrp * c.group);
        it.row0 = it.tile * rows_item;
        it.nrows = min(rows_item, G.rows_e - it.row0);
        return it;
    };

    // This wave's share of an item's loads: load k = wv + 16 j moves staged
    // bytes 1024 k + 16 lane of its part (row b / pitch, column b % pitch);
    // loads past the item write the sink.
    const Cursor c_first = cursor_at(i_begin);
    Cursor c_issue = c_first;
    int i_issue = i_begin;  // item the issue cursor points at
    auto issue = [&](int slot, int i) {  // items are issued in order
        uint32_t base = kMaskedOffset;
        int nrows = 0;
        if (i < i_end) {
            for (; i_issue < i; i_issue++) step(c_issue);
            const Item it = item_of(c_issue);
            base = (uint32_t)(((int64_t)it.e * G.rows_e + it.row0) * G.stride + (int64_t)it.half * G.row_bytes);
            nrows = it.nrows;
        }
        base = __builtin_amdgcn_readfirstlane(base);
        nrows = __builtin_amdgcn_readfirstlane(nrows);
#pragma unroll
        for (int j = 0; j < kMoDmaPerWave; j++) {
            const int k = wv + kMoWaves * j;
            const bool second = MODE == 0 && k >= G.part_dma;  // uniform
            const uint32_t b = 1024u * (uint32_t)(second ? k - G.part_dma : k) + 16u * lane;
            const uint32_t r = b / G.pitch, col = b - r * G.pitch;
            const bool ok = k < G.ndma && r < (uint32_t)nrows && col < G.row_bytes && base != kMaskedOffset;
            uint8_t *dst = k < G.ndma ? ring + slot * kMoSlot + 1024 * k : ring + kMoSlots * kMoSlot;
            __builtin_amdgcn_raw_ptr_buffer_load_lds(second ? rs1 : rs0, (lds_ptr)dst, 16,
                                                     ok ? base + r * G.stride + col : kMaskedOffset,
                                                     0, 0, kStreamLoad);
        }
    };

    // Wave roles.
    const int nwork = MODE == 0 ? 2 * G.nsb : G.rt * G.nsb;
    const bool active = wv < nwork;  // uniform
    const int sb = MODE == 0 ? wv % G.nsb : wv % G.nsb;
    const int mat = MODE == 0 ? wv / G.nsb : 0;
    const int rtile = MODE == 0 ? 0 : wv / G.nsb;
    const int n = lane & 15, g = lane >> 4, h = (lane >> 4) & 1, tq = lane >> 5;
    const uint32_t part_off = (uint32_t)(G.part_dma * 1024);
    const uint32_t ring_base = (uint32_t)(uintptr_t)(lds_ptr)ring;
    const uint32_t a_h0 = ring_base + mat * part_off + (rtile * 16 + n) * G.pitch + sb * PB;
    const uint32_t a_q0 = a_h0 + 16 + 8 * g;
    const i32x4 zero4 = {0, 0, 0, 0};

    // Operands of the current route group: A per MFMA pair and chunk; per
    // output lane the sub-block sums and the superblock scale of its route.
    // HV = 2: [0] for the first half's superblock sb, [1] for sb + nsb; A is
    // kept as the lane's two live dwords (Ac; rows m hold them in dwords
    // 0, 1 when (m >> 2) & 1 == 0, else in 2, 3), expanded at the MFMA, and
    // the sub-block sums and scales stay in the wave's scratch (9 floats at
    // 768 + 36 (4 half + route)), read per pair.
    i32x4 A[2][4];       // HV = 1
    uint2 Ac[HV][2][4];  // HV = 2
    float xs4[2][4], xs[2];  // HV = 1
    int cur_key = -1;  // e * 65536 + group of the operands held

    // Digits of route group `it` for this wave's superblock.
    // `between` runs after the vector loads are issued and before they are
    // used: in the prologue it issues the first items' loads, so the wait for
    // the vectors (issued first) does not wait for those.  Mid-stream
    // (drain = true) the vectors queue behind the ring's loads anyway.
    auto build = [&](const Item &it, bool drain, auto &&between) {
#pragma unroll
        for (int hf = 0; hf < HV; hf++) {
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    if constexpr (HV == 1) {
                        A[pp][c] = i32x4{0, 0, 0, 0};
                        xs4[pp][c] = 0.0f;
                    } else {
                        Ac[hf][pp][c] = uint2{0u, 0u};
                    }
                }
                if constexpr (HV == 1) xs[pp] = 0.0f;
            }
        }
        if (!active) {
            between();
            return;
        }
        const uint32_t sbase = (uint32_t)(uintptr_t)(lds_ptr)scratch[wv];
        int vrow[kGrp];  // vector row of each route
#pragma unroll
        for (int j = 0; j < kGrp; j++) {
            const int p = pairs[offsets[it.e] + kGrp * it.group + min(j, it.ntok - 1)];
            vrow[j] = MODE == 0 ? p / top_k : p;
        }
        // route ids for the reductions (lane-indexed: four constant LDS
        // addresses would each hold a register across the item loop)
        if (wv == 0 && lane < kGrp)
            gid[lane] = pairs[offsets[it.e] + kGrp * it.group + min(lane, it.ntok - 1)];
        // A half at a time (HV = 2: the second half's vectors are loaded once
        // the first half's digits are built, which keeps the registers in
        // bounds; their wait also covers the ring loads issued before them).
#pragma unroll
        for (int hf = 0; hf < HV; hf++) {
        float4 v[kGrp];
        // loads first, then one wait (this also drains the ring's loads)
#pragma unroll
        for (int j = 0; j < kGrp; j++)
            v[j] = reinterpret_cast<const float4 *>(vec + (int64_t)vrow[j] * G.vec_len + (sb + hf * G.nsb) * kQK)[lane];
        if (hf == 0) between();
        if (drain || hf > 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // Consume every loaded vector so the compiler's own wait comes here
        // (it cannot see the one above): a load it still thought outstanding
        // would make it wait for all loads before the next write of its registers.
        if constexpr (kGrp == 2)
            asm volatile("" ::"v"(v[0].x), "v"(v[1].x));
        else
            asm volatile("" ::"v"(v[0].x), "v"(v[1].x), "v"(v[2].x), "v"(v[3].x));
#pragma unroll
        for (int j = 0; j < kGrp; j++) {
            if (j >= it.ntok) break;  // uniform
            const float vv[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
            uint32_t mb = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) mb = max(mb, __float_as_uint(vv[k]) & 0x7FFFFFFFu);
            mb = wave_max_u32(mb);
            const bool finite = mb < 0x7F800000u;
            int ex = 0;
            (void)frexpf(__uint_as_float(mb), &ex);
            uint32_t d0 = 0, d1 = 0, d2 = 0;
            int sx = 0;
#pragma unroll
            for (int k = 0; k < 4; k++) {
                const int X = finite ? (int)rintf(ldexpf(vv[k], 22 - ex)) : 0;  // |X| <= 2^22
                const int c0 = (int)(int8_t)(X & 0xFF);
                const int X1 = (X - c0) >> 8;
                const int c1 = (int)(int8_t)(X1 & 0xFF);
                const int c2 = (X1 - c1) >> 8;
                d0 |= ((uint32_t)c0 & 0xFFu) << (8 * k);
                d1 |= ((uint32_t)c1 & 0xFFu) << (8 * k);
                d2 |= ((uint32_t)c2 & 0xFFu) << (8 * k);
                sx += X;
            }
            if constexpr (WT == kQ6_K) {  // sums over 16 elements (four lanes)
                sx += dpp_i<0xB1>(sx);
                sx += dpp_i<0x4E>(sx);
            } else {
                sx = sum8_i(sx);
            }
            const float scale = finite ? ldexpf(1.0f, ex - 22) : __builtin_nanf("");
            // scratch: planes at 0 / 256 / 512, sub-block sums (fp32) at 768 + 4 j
            // (Q6_K: 16-element sums at 768 + 4 quarter), scale at 832
            asm volatile(
                "ds_write_b32 %0, %1\n\t"
                "ds_write_b32 %0, %2 offset:256\n\t"
                "ds_write_b32 %0, %3 offset:512"
                :
                : "v"(sbase + 4 * lane), "v"(d0), "v"(d1), "v"(d2)
                : "memory");
            if constexpr (WT == kQ6_K) {
                if ((lane & 3) == 0)
                    asm volatile("ds_write_b32 %0, %1 offset:768"
                                 :
                                 : "v"(sbase + 4 * (lane >> 2)), "v"(__float_as_int((float)sx * scale))
                                 : "memory");
                if (lane == 0)
                    asm volatile("ds_write_b32 %0, %1 offset:832" : : "v"(sbase), "v"(__float_as_int(scale)) : "memory");
            } else if constexpr (HV == 1) {
                if ((lane & 7) == 0)
                    asm volatile("ds_write_b32 %0, %1 offset:768"
                                 :
                                 : "v"(sbase + 4 * (lane >> 3)), "v"(__float_as_int((float)sx * scale))
                                 : "memory");
                if (lane == 0)
                    asm volatile("ds_write_b32 %0, %1 offset:832" : : "v"(sbase), "v"(__float_as_int(scale)) : "memory");
            } else {  // kept for the items: sums at + 4 sub-block, scale at + 32
                // the slot offset enters through an asm so its address is
                // formed here, not kept in a register across the item loop
                uint32_t so = 768u + 36u * (uint32_t)(4 * hf + j);
                asm volatile("" : "+v"(so));
                const uint32_t slot = sbase + so;
                if ((lane & 7) == 0)
                    asm volatile("ds_write_b32 %0, %1"
                                 :
                                 : "v"(slot + 4 * (lane >> 3)), "v"(__float_as_int((float)sx * scale))
                                 : "memory");
                if (lane == 0)
                    asm volatile("ds_write_b32 %0, %1 offset:32" : : "v"(slot), "v"(__float_as_int(scale)) : "memory");
            }
            if constexpr (WT == kQ6_K) {
                // Q6_K: one route per MFMA.  Chunk c covers elements 128 (c >> 1)
                // + 32 (c & 1) + l and + 64 (l < 32); A row m = 4 q + p holds
                // plane p < 3 of quarter q (16 elements), live on the lanes g
                // with g >> 1 == q & 1, in bytes 0..7 (q < 2, l = 8 g ..) or
                // 8..15 (q >= 2, + 64).  Output lane n + 16 g: quarter g, whose
                // sum of x is quarter 8 (c >> 1) + 2 (c & 1) + 4 (g >> 1) + (g & 1).
                const int m = lane & 15, p = m & 3, q = m >> 2;
                uint2 lo[4], hi[4];
                float xq[4], sc;
                asm volatile(
                    "ds_read_b64 %0, %13\n\t"
                    "ds_read_b64 %1, %13 offset:32\n\t"
                    "ds_read_b64 %2, %13 offset:128\n\t"
                    "ds_read_b64 %3, %13 offset:160\n\t"
                    "ds_read_b64 %4, %13 offset:64\n\t"
                    "ds_read_b64 %5, %13 offset:96\n\t"
                    "ds_read_b64 %6, %13 offset:192\n\t"
                    "ds_read_b64 %7, %13 offset:224\n\t"
                    "ds_read_b32 %8, %14 offset:768\n\t"
                    "ds_read_b32 %9, %14 offset:776\n\t"
                    "ds_read_b32 %10, %14 offset:800\n\t"
                    "ds_read_b32 %11, %14 offset:808\n\t"
                    "ds_read_b32 %12, %15 offset:832\n\t"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(lo[0]), "=&v"(lo[1]), "=&v"(lo[2]), "=&v"(lo[3]), "=&v"(hi[0]), "=&v"(hi[1]),
                      "=&v"(hi[2]), "=&v"(hi[3]), "=&v"(xq[0]), "=&v"(xq[1]), "=&v"(xq[2]), "=&v"(xq[3]), "=&v"(sc)
                    : "v"(sbase + (p < 3 ? p : 0) * 256 + 8 * g), "v"(sbase + 16 * (g >> 1) + 4 * (g & 1)),
                      "v"(sbase)
                    : "memory");
                const bool lo_live = p < 3 && q == (g >> 1), hi_live = p < 3 && q == 2 + (g >> 1);
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    A[j][c] = i32x4{lo_live ? (int)lo[c].x : 0, lo_live ? (int)lo[c].y : 0,
                                    hi_live ? (int)hi[c].x : 0, hi_live ? (int)hi[c].y : 0};
                    xs4[j][c] = xq[c];
                }
                xs[j] = sc;
                continue;
            }
            // A rows of route j: m = 8 (j & 1) + 4 ha + p in lanes m + 16 g; this
            // output lane's sub-blocks 2 c + h.
            const int m = lane & 15, p = m & 3, ha = (m >> 2) & 1;
            uint2 dl[4], dh[4];
            float xsv[4], sc;
            asm volatile(
                "ds_read_b64 %0, %13\n\t"
                "ds_read_b64 %1, %13 offset:64\n\t"
                "ds_read_b64 %2, %13 offset:128\n\t"
                "ds_read_b64 %3, %13 offset:192\n\t"
                "ds_read_b64 %4, %13 offset:32\n\t"
                "ds_read_b64 %5, %13 offset:96\n\t"
                "ds_read_b64 %6, %13 offset:160\n\t"
                "ds_read_b64 %7, %13 offset:224\n\t"
                "ds_read_b32 %8, %14 offset:768\n\t"
                "ds_read_b32 %9, %14 offset:776\n\t"
                "ds_read_b32 %10, %14 offset:784\n\t"
                "ds_read_b32 %11, %14 offset:792\n\t"
                "ds_read_b32 %12, %15 offset:832\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(dl[0]), "=&v"(dl[1]), "=&v"(dl[2]), "=&v"(dl[3]), "=&v"(dh[0]), "=&v"(dh[1]),
                  "=&v"(dh[2]), "=&v"(dh[3]), "=&v"(xsv[0]), "=&v"(xsv[1]), "=&v"(xsv[2]), "=&v"(xsv[3]),
                  "=&v"(sc)
                : "v"(sbase + (p < 3 ? p : 0) * 256 + 8 * g), "v"(sbase + 4 * h), "v"(sbase)
                : "memory");
            const int pp = j >> 1, tj = j & 1;
            const bool mine_in = ((m >> 3) == tj) && p < 3;  // A row of route j, live plane
#pragma unroll
            for (int c = 0; c < 4; c++) {
                if (mine_in) {
                    if constexpr (HV == 1)
                        A[pp][c] = i32x4{ha == 0 ? (int)dl[c].x : 0, ha == 0 ? (int)dl[c].y : 0,
                                         ha == 1 ? (int)dh[c].x : 0, ha == 1 ? (int)dh[c].y : 0};
                    else
                        Ac[hf][pp][c] = ha == 0 ? dl[c] : dh[c];
                }
            }
            if (HV == 1 && tq == tj) {  // output lanes of route j
#pragma unroll
                for (int c = 0; c < 4; c++) xs4[pp][c] = xsv[c];
                xs[pp] = sc;
            }
        }
        }  // halves
    };

    // Results of item `it` from the partial sums in part[buf]: one wave per item.
    int nout = 0;  // buffered results (every wave keeps the same count)
    auto reduce = [&](const Item &it, int buf, int base) {
        if (MODE == 0) {
            // the lane's LDS addresses are formed here, not kept live across
            // the item loop
            int ln = lane;
            asm volatile("" : "+v"(ln));
            if (ln < it.ntok * 16) {
                const int tk = ln >> 4, r = ln & 15;
                if (r < it.nrows) {
                    // the second half continues the first half's sums
                    float gs = HV == 2 && it.half == 1 ? hsave[ln][0] : 0.0f;
                    float us = HV == 2 && it.half == 1 ? hsave[ln][1] : 0.0f;
                    for (int s = 0; s < G.nsb; s++) {
                        gs += part[buf][tk][s][r];
                        us += part[buf][tk][G.nsb + s][r];
                    }
                    if (HV == 2 && it.half == 0) {  // uniform: no result yet
                        hsave[ln][0] = gs;
                        hsave[ln][1] = us;
                        return;
                    }
                    const int p = gid[tk];
                    const int slot = base + tk * it.nrows + r;
                    outv[slot] = gs / (1.0f + expf(-gs)) * us;  // silu(gate) * up
                    outi[slot] = p * G.out_len + it.row0 + r;
                }
            }
        } else {
            for (int q = lane; q < it.ntok * rows_item; q += 64) {
                const int tk = q / rows_item, r = q - tk * rows_item;
                if (r < it.nrows) {
                    const int t16 = r >> 4, rr = r & 15;
                    float ys = 0.0f;
                    for (int s = 0; s < G.nsb; s++) ys += part[buf][tk][t16 * G.nsb + s][rr];
                    const int p = gid[tk];
                    const int slot = base + tk * it.nrows + r;
                    outv[slot] = ys;
                    outi[slot] = p * G.out_len + it.row0 + r;
                }
            }
        }
    };
    // The reduction of the previous item by its wave; every wave advances nout.
    auto reduce_prev = [&](const Item &it, int i_prev) {
        if (wv == i_prev % kMoWaves) reduce(it, i_prev & 1, nout);
        if (HV == 1 || it.half == HV - 1) nout += it.ntok * it.nrows;
    };
    auto flush = [&]() {
        __syncthreads();
        if constexpr (REC) {
            // Buffered h come in runs of 16 (one route's 16-row group), each
            // a row of 16 lanes: converted to records here.
            for (int q = threadIdx.x; q < nout; q += kMoThreads) {
                const int r = q & 15, rg = outi[q] >> 4;
                float scale, sum;
                const uint32_t rec = h_record16(outv[q], scale, sum);
                float *o = out + kRecDwords * rg;
                if ((r & 3) < 3) o[4 * (r & 3) + (r >> 2)] = __uint_as_float(rec);
                if (r < 2) o[12 + r] = r == 0 ? scale : sum;
            }
        } else {
            for (int q = threadIdx.x; q < nout; q += kMoThreads) out[outi[q]] = outv[q];
        }
        nout = 0;
        __syncthreads();
    };

    // Prologue: the first item's loads, the first group's vectors, the next
    // items' loads, then the group's operands.  Every workgroup starts at
    // once, and the memory system serves requests issued together
    // interleaved: issued first, item 0 lands well before the items after it
    // instead of together with them.
    Cursor c_cur = c_first;
    Item cur = item_of(c_cur);
    issue(0, i_begin);
    build(cur, false, [&]() {
#pragma unroll
        for (int j = 1; j < kMoSlots - 1; j++) issue(j, i_begin + j);
    });
    cur_key = cur.e * 65536 + cur.group;

    int slot = 0;
    Item prev = cur;
    bool have_prev = false;
    for (int i = i_begin; i < i_end; i++) {
        if (i > i_begin) step(c_cur);
        cur = item_of(c_cur);
        const int key = cur.e * 65536 + cur.group;
        const bool rebuild = key != cur_key;  // uniform
        if (rebuild) {
            // The previous item's results, then every buffered result, then
            // the new operands (whose loads drain the ring's loads).
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (have_prev) reduce_prev(prev, i - 1);
            have_prev = false;
            flush();
            build(cur, true, []() {});
            cur_key = key;
        }
        if (!rebuild && nout + 2 * kMoGroup * rows_item > kMoOutCap) {
            asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
            if (have_prev) reduce_prev(prev, i - 1);
            have_prev = false;
            flush();
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        }
        asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(kMoDmaPerWave * (kMoSlots - 2)) : "memory");
        if (have_prev) reduce_prev(prev, i - 1);
        issue(slot == 0 ? kMoSlots - 1 : slot - 1, i + kMoSlots - 1);
        if constexpr (WT == kQ6_K) {
            if (active) {
                // Q6_K rows (210-byte superblocks: ql[128], qh[64], 16 int8
                // scales, d), 0 or 2 bytes past a dword in the slot: aligned
                // dwords, realigned.  Chunk c = (half c >> 1, part c & 1) is ql
                // bytes 32 c + l, low nibbles for elements 128 (c >> 1) + 32 (c &
                // 1) + l and high nibbles for + 64, the two high bits from qh
                // byte 32 (c >> 1) + l (bits 2 (c & 1), and 4 + 2 (c & 1)); lane
                // group g takes l = 8 g .. 8 g + 7 as B bytes 0..7 and 8..15.
                // Codes q = 0..63 against one route's x digits per MFMA; output
                // lane n + 16 g holds quarter g's plane sums, whose sum q X can
                // reach 16 * 63 * 2^22 and so combine in fp32.  value = d sum
                // sc (xs S - 32 X) over the quarters, the reference's d sc (q -
                // 32) per element.
                const uint32_t sa = a_h0 + (uint32_t)slot * kMoSlot;
                const uint32_t sh = sa & 3u, ab = sa - sh, aq = ab + 8u * (uint32_t)g;
                uint2 p01[6], s01, s23;
                uint32_t p2[6], s4;
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
                const uint32_t s0 = __builtin_amdgcn_alignbyte(s01.y, s01.x, sh);
                const uint32_t s1 = __builtin_amdgcn_alignbyte(s23.x, s01.y, sh);
                const uint32_t s2 = __builtin_amdgcn_alignbyte(s23.y, s23.x, sh);
                const uint32_t s3 = __builtin_amdgcn_alignbyte(s4, s23.y, sh);
                const float d = half_bits_to_float_fast(s4 >> (8 * sh));
                i32x4 B[4];
                float scq[4];
                // quarter g's scale: byte 2 (c & 1) + (g & 1) of scale dword 2 (c >> 1) + (g >> 1)
                const uint32_t slo = (g >> 1) ? s1 : s0, shi = (g >> 1) ? s3 : s2;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int ip = c >> 1, pt = c & 1;
                    uint32_t b[4];
#pragma unroll
                    for (int k = 0; k < 2; k++) {
                        const uint32_t hq = qh[ip][k];
                        b[k] = (ql[c][k] & 0x0F0F0F0Fu) | ((pt == 0 ? hq << 4 : hq << 2) & 0x30303030u);
                        b[2 + k] = ((ql[c][k] >> 4) & 0x0F0F0F0Fu) | ((pt == 0 ? hq : hq >> 2) & 0x30303030u);
                    }
                    B[c] = i32x4{(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
                    const uint32_t sw = ip ? shi : slo;
                    scq[c] = (float)(int)(int8_t)((sw >> (8 * ((g & 1) + 2 * pt))) & 0xFFu);
                }
#pragma unroll
                for (int j = 0; j < kGrp; j++) {
                    if (j >= cur.ntok) break;  // uniform
                    i32x4 D[4];
#pragma unroll
                    for (int c = 0; c < 4; c++) D[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[j][c], B[c], zero4, 0, 0, 0);
                    float v = 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        const float S = fmaf((float)D[c][2], 65536.0f, (float)(D[c][0] + 256 * D[c][1]));
                        v = fmaf(scq[c], fmaf(S, xs[j], -32.0f * xs4[j][c]), v);
                    }
                    v *= d;
                    v += __shfl_xor(v, 16);
                    v += __shfl_xor(v, 32);
                    if (g == 0) part[i & 1][j][wv][n] = v;
                }
            }
        } else if (active && WT == kQ4_0) {
            // Q4_0: a 144-byte piece is eight 18-byte blocks; chunk c (64
            // columns) is blocks 2c and 2c + 1.  Lane group g takes elements
            // 8 g .. 8 g + 7 of each: quant bytes 8 (g & 1) .. + 7 of the
            // block, nibble g >> 1 (elements 16 .. 31 are the high nibbles),
            // so B = {block 2c's 8 codes, block 2c + 1's 8 codes} as bytes
            // 0..15 against A's {elements 64c + 8g .., 64c + 32 + 8g ..}.
            // Output half h (= g & 1) sums block 2c + h; its d is read with
            // the codes.  value = sum_c d_(2c+h) (scale S_c - 8 sum x), the
            // reference's d * sum((q - 8) x) per block.
            const uint32_t off = (uint32_t)slot * kMoSlot;
            const uint32_t pbase = a_h0 + off;            // row n's piece
            const uint32_t qb = pbase + 8u * (uint32_t)h;  // + quant offset 8 (g & 1)
            const uint32_t db = pbase + 16u * (uint32_t)h; // d of block 2c + h at + 36 c (half h)
            uint32_t w[4][3], v[4][2], dd[4];
            asm volatile(
                "ds_read_b32 %0, %24\n\t"
                "ds_read_b32 %1, %24 offset:4\n\t"
                "ds_read_b32 %2, %24 offset:8\n\t"
                "ds_read_b32 %3, %24 offset:20\n\t"
                "ds_read_b32 %4, %24 offset:24\n\t"
                "ds_read_b32 %5, %25\n\t"
                "ds_read_b32 %6, %24 offset:36\n\t"
                "ds_read_b32 %7, %24 offset:40\n\t"
                "ds_read_b32 %8, %24 offset:44\n\t"
                "ds_read_b32 %9, %24 offset:56\n\t"
                "ds_read_b32 %10, %24 offset:60\n\t"
                "ds_read_b32 %11, %25 offset:36\n\t"
                "ds_read_b32 %12, %24 offset:72\n\t"
                "ds_read_b32 %13, %24 offset:76\n\t"
                "ds_read_b32 %14, %24 offset:80\n\t"
                "ds_read_b32 %15, %24 offset:92\n\t"
                "ds_read_b32 %16, %24 offset:96\n\t"
                "ds_read_b32 %17, %25 offset:72\n\t"
                "ds_read_b32 %18, %24 offset:108\n\t"
                "ds_read_b32 %19, %24 offset:112\n\t"
                "ds_read_b32 %20, %24 offset:116\n\t"
                "ds_read_b32 %21, %24 offset:128\n\t"
                "ds_read_b32 %22, %24 offset:132\n\t"
                "ds_read_b32 %23, %25 offset:108\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(w[0][0]), "=&v"(w[0][1]), "=&v"(w[0][2]), "=&v"(v[0][0]), "=&v"(v[0][1]), "=&v"(dd[0]),
                  "=&v"(w[1][0]), "=&v"(w[1][1]), "=&v"(w[1][2]), "=&v"(v[1][0]), "=&v"(v[1][1]), "=&v"(dd[1]),
                  "=&v"(w[2][0]), "=&v"(w[2][1]), "=&v"(w[2][2]), "=&v"(v[2][0]), "=&v"(v[2][1]), "=&v"(dd[2]),
                  "=&v"(w[3][0]), "=&v"(w[3][1]), "=&v"(w[3][2]), "=&v"(v[3][0]), "=&v"(v[3][1]), "=&v"(dd[3])
                : "v"(qb), "v"(db)
                : "memory");
            const uint32_t nib = 4u * (uint32_t)tq;  // g >> 1
            i32x4 B[4];
            float dq[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                // block 2c's codes start 2 bytes into the first dword
                const uint32_t b0 = __builtin_amdgcn_alignbyte(w[c][1], w[c][0], 2);
                const uint32_t b1 = __builtin_amdgcn_alignbyte(w[c][2], w[c][1], 2);
                B[c] = i32x4{(int)((b0 >> nib) & 0x0F0F0F0Fu), (int)((b1 >> nib) & 0x0F0F0F0Fu),
                             (int)((v[c][0] >> nib) & 0x0F0F0F0Fu), (int)((v[c][1] >> nib) & 0x0F0F0F0Fu)};
                dq[c] = half_bits_to_float_fast(h ? dd[c] >> 16 : dd[c] & 0xFFFFu);
            }
            const int npairs = (cur.ntok + 1) >> 1;
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                if (pp >= npairs) break;  // uniform
                i32x4 D[4];
#pragma unroll
                for (int c = 0; c < 4; c++) D[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[pp][c], B[c], zero4, 0, 0, 0);
                float val = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    const int S = (int)(((uint32_t)D[c][2] << 16) + (((uint32_t)D[c][1] << 8) + (uint32_t)D[c][0]));
                    val = fmaf(dq[c], fmaf(xs[pp], (float)S, -8.0f * xs4[pp][c]), val);
                }
                const float other = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(val), 0x401F));
                if (h == 0) part[i & 1][2 * pp + tq][wv][n] = val + other;
            }
        } else if (active) {
            u32x4 hv;
            uint2 q[4], qh;
            const uint32_t off = (uint32_t)slot * kMoSlot;
            if constexpr (WT == kQ5_K) {
                // Q5_K: header, then qh (32 bytes: bit 2c / 2c + 1 of byte i
                // is the fifth bit of element i of sub-blocks 2c / 2c + 1),
                // then the quants at + 48
                asm volatile(
                    "ds_read_b128 %0, %6\n\t"
                    "ds_read_b64 %1, %7 offset:32\n\t"
                    "ds_read_b64 %2, %7 offset:64\n\t"
                    "ds_read_b64 %3, %7 offset:96\n\t"
                    "ds_read_b64 %4, %7 offset:128\n\t"
                    "ds_read_b64 %5, %7\n\t"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(hv), "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3]), "=&v"(qh)
                    : "v"(a_h0 + off), "v"(a_q0 + off)
                    : "memory");
            } else {
                asm volatile(
                    "ds_read_b128 %0, %5\n\t"
                    "ds_read_b64 %1, %6\n\t"
                    "ds_read_b64 %2, %6 offset:32\n\t"
                    "ds_read_b64 %3, %6 offset:64\n\t"
                    "ds_read_b64 %4, %6 offset:96\n\t"
                    "s_waitcnt lgkmcnt(0)"
                    : "=&v"(hv), "=&v"(q[0]), "=&v"(q[1]), "=&v"(q[2]), "=&v"(q[3])
                    : "v"(a_h0 + off), "v"(a_q0 + off)
                    : "memory");
            }
            i32x4 B[4];
#pragma unroll
            for (int c = 0; c < 4; c++) {
                uint32_t l0 = q[c].x & 0x0F0F0F0Fu, l1 = q[c].y & 0x0F0F0F0Fu;
                uint32_t h0 = (q[c].x >> 4) & 0x0F0F0F0Fu, h1 = (q[c].y >> 4) & 0x0F0F0F0Fu;
                if constexpr (WT == kQ5_K) {  // codes 0..31
                    l0 |= ((qh.x >> (2 * c)) & 0x01010101u) << 4;
                    l1 |= ((qh.y >> (2 * c)) & 0x01010101u) << 4;
                    h0 |= ((qh.x >> (2 * c + 1)) & 0x01010101u) << 4;
                    h1 |= ((qh.y >> (2 * c + 1)) & 0x01010101u) << 4;
                }
                B[c] = i32x4{(int)l0, (int)l1, (int)h0, (int)h1};
            }
            // The plane sums combined (a sub-block's 32 products): exactly in
            // int32 for Q4_K (|sum q X| <= 32 * 15 * 2^22 < 2^31); in fp32 for
            // Q5_K, whose 32 * 31 * 2^22 does not fit (two roundings, relative
            // error under 2^-23).
            auto plane_sum = [](const i32x4 &Dc) {
                if constexpr (WT == kQ5_K)
                    return fmaf((float)Dc[2], 65536.0f, (float)(Dc[0] + 256 * Dc[1]));
                else
                    return (float)(int)(((uint32_t)Dc[2] << 16) + (((uint32_t)Dc[1] << 8) + (uint32_t)Dc[0]));
            };
            const float d = half_bits_to_float_fast(hv.x);
            const float dmin = half_bits_to_float_fast(hv.x >> 16);
            // 6-bit codes (RT/GgufKQuantLayout.java:37-49) of sub-blocks h, 2 + h, 4 + h, 6 + h
            const uint32_t hy = hv.y >> (8 * h), hz = hv.z >> (8 * h), hw = hv.w >> (8 * h);
            const uint32_t sc03 = hy & 0x003F003Fu;
            const uint32_t mn03 = hz & 0x003F003Fu;
            const uint32_t sc47 = (hw & 0x000F000Fu) | ((hy >> 2) & 0x00300030u);
            const uint32_t mn47 = ((hw >> 4) & 0x000F000Fu) | ((hz >> 2) & 0x00300030u);
            const float scf[4] = {(float)(sc03 & 0xFFu), (float)((sc03 >> 16) & 0xFFu),
                                  (float)(sc47 & 0xFFu), (float)((sc47 >> 16) & 0xFFu)};
            const float mnf[4] = {(float)(mn03 & 0xFFu), (float)((mn03 >> 16) & 0xFFu),
                                  (float)(mn47 & 0xFFu), (float)((mn47 >> 16) & 0xFFu)};
            const bool fin = __builtin_isfinite(d) && __builtin_isfinite(dmin);
            const int npairs = (cur.ntok + 1) >> 1;
            // the half's operands by a compile-time index (a runtime pick of a
            // register array would go through scratch)
            const bool lo_dw = ((n >> 2) & 1) == 0;  // this lane's A row holds dwords 0, 1
            // HV = 2: this lane's slot bases (route tq + 2 pp at + 72 pp + 144 half)
            const uint32_t xl_s = (uint32_t)(uintptr_t)(lds_ptr)scratch[wv] + 36u * (uint32_t)tq;
            const uint32_t xl_h = xl_s + 4u * (uint32_t)h;
            // (half, pair) by compile-time indices: register arrays and LDS
            // offsets stay fixed (a runtime index would go through scratch)
            auto pairs_of = [&](auto hfc, auto ppc) {
            constexpr int hf = decltype(hfc)::value, pp = decltype(ppc)::value;
            {
                if (pp >= npairs) return;  // uniform
                // route 2 pp + tq's sums of sub-blocks 2 c + h and its scale
                float xs4h[4], xsh;
                if constexpr (HV == 1) {
#pragma unroll
                    for (int c = 0; c < 4; c++) xs4h[c] = xs4[pp][c];
                    xsh = xs[pp];
                } else {
                    constexpr int so = 768 + 36 * (4 * hf + 2 * pp);
                    asm volatile(
                        "ds_read_b32 %0, %5 offset:%7\n\t"
                        "ds_read_b32 %1, %5 offset:%8\n\t"
                        "ds_read_b32 %2, %5 offset:%9\n\t"
                        "ds_read_b32 %3, %5 offset:%10\n\t"
                        "ds_read_b32 %4, %6 offset:%11\n\t"
                        "s_waitcnt lgkmcnt(0)"
                        : "=&v"(xs4h[0]), "=&v"(xs4h[1]), "=&v"(xs4h[2]), "=&v"(xs4h[3]), "=&v"(xsh)
                        : "v"(xl_h), "v"(xl_s), "n"(so), "n"(so + 8), "n"(so + 16), "n"(so + 24), "n"(so + 32)
                        : "memory");
                }
                // the pair's four products first, then their plane combines
                i32x4 D[4];
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    i32x4 a;
                    if constexpr (HV == 1) {
                        a = A[pp][c];
                    } else {
                        const int u0 = (int)Ac[hf][pp][c].x, u1 = (int)Ac[hf][pp][c].y;
                        a = lo_dw ? i32x4{u0, u1, 0, 0} : i32x4{0, 0, u0, u1};
                    }
                    D[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, B[c], zero4, 0, 0, 0);
                }
                float S[4];
#pragma unroll
                for (int c = 0; c < 4; c++) S[c] = plane_sum(D[c]);
                float v;
                if (fin) {
                    float qs = 0.0f, mm = 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        qs = fmaf(scf[c], S[c], qs);
                        mm = fmaf(mnf[c], xs4h[c], mm);
                    }
                    v = fmaf(d * xsh, qs, -(dmin * mm));
                } else {
                    // the reference's (d sc) products; zero min codes skip a
                    // non-finite dmin (minContribution, RT/GgufKQuantLayout.java:67-69)
                    float qs = 0.0f, mm = 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        qs = fmaf(d * scf[c], xsh * S[c], qs);
                        mm = fmaf(mnf[c] != 0.0f ? dmin * mnf[c] : 0.0f, xs4h[c], mm);
                    }
                    v = qs - mm;
                }
                // h = 1 half of row n: lane n + 16 (ds_swizzle, lanes xor 16)
                const float other = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
                if (h == 0) part[i & 1][2 * pp + tq][wv][n] = v + other;
            }
            };
            if constexpr (HV == 2) {
                if (cur.half == 1) {  // uniform
                    pairs_of(std::integral_constant<int, 1>{}, std::integral_constant<int, 0>{});
                    pairs_of(std::integral_constant<int, 1>{}, std::integral_constant<int, 1>{});
                } else {
                    pairs_of(std::integral_constant<int, 0>{}, std::integral_constant<int, 0>{});
                    pairs_of(std::integral_constant<int, 0>{}, std::integral_constant<int, 1>{});
                }
            } else {  // one half: the pairs in a loop (the form the hidden <= 2048 passes were tuned in)
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                if (pp >= npairs) break;  // uniform
                // the pair's four products first, then their plane combines
                i32x4 D[4];
#pragma unroll
                for (int c = 0; c < 4; c++) D[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[pp][c], B[c], zero4, 0, 0, 0);
                float S[4];
#pragma unroll
                for (int c = 0; c < 4; c++) S[c] = plane_sum(D[c]);
                float v;
                if (fin) {
                    float qs = 0.0f, mm = 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        qs = fmaf(scf[c], S[c], qs);
                        mm = fmaf(mnf[c], xs4[pp][c], mm);
                    }
                    v = fmaf(d * xs[pp], qs, -(dmin * mm));
                } else {
                    // the reference's (d sc) products; zero min codes skip a
                    // non-finite dmin (minContribution, RT/GgufKQuantLayout.java:67-69)
                    float qs = 0.0f, mm = 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        qs = fmaf(d * scf[c], xs[pp] * S[c], qs);
                        mm = fmaf(mnf[c] != 0.0f ? dmin * mnf[c] : 0.0f, xs4[pp][c], mm);
                    }
                    v = qs - mm;
                }
                // h = 1 half of row n: lane n + 16 (ds_swizzle, lanes xor 16)
                const float other = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
                if (h == 0) part[i & 1][2 * pp + tq][wv][n] = v + other;
            }
            }
                }
        prev = cur;
        have_prev = true;
        slot = slot == kMoSlots - 1 ? 0 : slot + 1;
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if (have_prev) reduce_prev(prev, i_end - 1);
    flush();
}

// ---- Down projection and combine, token-major --------------------------
//
// Workgroup = (16 rows of H, group of tg tokens): wave 0 groups the
// workgroup's tg * top_k <= 64 routes by expert (items); wave w takes items
// w, w + waves, ... and works through their routes one unit (item, route)
// at a time.  A unit's loads are the item's 16-row down tile (16 x I/256
// superblocks, into one of the wave's three tile slots; a later unit of the
// same item loads nothing there) and the route's h records (into one of
// three route slots); the loads of unit k + 2 go out before unit k is
// computed, so two units are in flight per wave and no wave waits on
// another until the combine.  A route's 16 results go to LDS; then every
// token's rows are combined in route order, fp32 multiply then add
// (MoeForwardPass.java:217-240, :461-472), skipping the routes
// moe_combine_kernel skips.
//
// Contraction (v_mfma_i32_16x16x64_i8, B = the tile's nibbles as in the
// GEMV): h records carry one power-of-two scale per 16 elements, so A row
// m = 4 q + p holds plane p < 3 of quarter q of the chunk (16 elements:
// half q & 1 of sub-block 2 c + (q >> 1)), live on the lanes g with
// g >> 1 == q & 1, in bytes 0..7 (q < 2, low nibbles) or 8..15; output lane
// n + 16 g holds the plane sums of row n and quarter g,
// D0 + 256 D1 + 65536 D2 = sum q X, exactly in int32 for Q4_K and Q5_K
// codes (|.| <= 16 * 31 * 2^22 < 2^31) and in fp32 for Q6_K's (up to
// 16 * 63 * 2^22), which it scales by the quarter's scale before the
// sub-block's d sc.
namespace {

constexpr int kMdMaxWaves = 8;
constexpr int kMdRoutes = 64;  // routes per workgroup
constexpr int kMdSlots = 2;    // tile and route slots per wave (units in flight + 1)

constexpr int kQ6KBlockBytes = 210;
// Down rows (type dt): Q4_K and Q5_K at a pitch of odd 16-byte units (the 16
// rows' reads spread over the banks); Q6_K packed as stored: a 16-row tile of
// 210-byte superblocks is one contiguous, 16-byte aligned run (16 x 210 = 3360).
constexpr uint32_t md_row_bytes(int nsb, int dt) {
    return nsb * (dt == kQ6_K ? kQ6KBlockBytes : dt == kQ5_K ? kQ5KBlockBytes : kQKBlockBytes);
}
constexpr uint32_t md_pitch(int nsb, int dt) {
    return dt == kQ6_K || (md_row_bytes(nsb, dt) / 16) % 2 == 1 ? md_row_bytes(nsb, dt) : md_row_bytes(nsb, dt) + 16;
}
// A slot's bytes move as whole kilobytes (16 bytes a lane) plus a tail of
// 256-byte loads (4 bytes a lane), so slots take no more LDS than they hold.
constexpr int md_tile_bytes(int nsb, int dt) { return 16 * (int)md_pitch(nsb, dt); }
constexpr int md_route_bytes(int nsb) { return nsb * 16 * kRecDwords * 4; }
constexpr int md_full(int bytes) { return bytes / 1024; }
constexpr int md_tail(int bytes) { return (bytes % 1024 + 255) / 256; }
constexpr int md_slot(int bytes) { return 1024 * md_full(bytes) + 256 * md_tail(bytes); }

}  // namespace

// One unit's LDS operands of superblock s: the 16 rows' header and quant
// bytes (B), the A halves (records or the zero sink) and (scale, sum).
struct MdSb {
    u32x4 hv;
    uint2 qb[4], xl[4], xh[4];
    float2 xp[4];
    uint2 qh;  // Q5_K: the lane's 8 qh bytes
};
// Reads of superblock s for one asm statement (named operands, so one
// statement can read every superblock of a unit and wait once).
#define MD_SB_READS(s)                                                                            \
    "ds_read_b128 %[hv" #s "], %[th" #s "]\n\t"                                                   \
    "ds_read_b64 %[qa" #s "], %[tq" #s "]\n\t"                                                    \
    "ds_read_b64 %[qb" #s "], %[tq" #s "] offset:32\n\t"                                          \
    "ds_read_b64 %[qc" #s "], %[tq" #s "] offset:64\n\t"                                          \
    "ds_read_b64 %[qd" #s "], %[tq" #s "] offset:96\n\t"                                          \
    "ds_read_b64 %[la" #s "], %[rl" #s "]\n\t"                                                    \
    "ds_read_b64 %[lb" #s "], %[rl" #s "] offset:224\n\t"                                         \
    "ds_read_b64 %[lc" #s "], %[rl" #s "] offset:448\n\t"                                         \
    "ds_read_b64 %[ld" #s "], %[rl" #s "] offset:672\n\t"                                         \
    "ds_read_b64 %[ha" #s "], %[rh" #s "]\n\t"                                                    \
    "ds_read_b64 %[hb" #s "], %[rh" #s "] offset:224\n\t"                                         \
    "ds_read_b64 %[hc" #s "], %[rh" #s "] offset:448\n\t"                                         \
    "ds_read_b64 %[hd" #s "], %[rh" #s "] offset:672\n\t"                                         \
    "ds_read_b64 %[pa" #s "], %[rp" #s "]\n\t"                                                    \
    "ds_read_b64 %[pb" #s "], %[rp" #s "] offset:224\n\t"                                         \
    "ds_read_b64 %[pc" #s "], %[rp" #s "] offset:448\n\t"                                         \
    "ds_read_b64 %[pd" #s "], %[rp" #s "] offset:672\n\t"
#define MD_SB_OUTS(s)                                                                             \
    [hv##s] "=&v"(o[s].hv), [qa##s] "=&v"(o[s].qb[0]), [qb##s] "=&v"(o[s].qb[1]),                  \
        [qc##s] "=&v"(o[s].qb[2]), [qd##s] "=&v"(o[s].qb[3]), [la##s] "=&v"(o[s].xl[0]),            \
        [lb##s] "=&v"(o[s].xl[1]), [lc##s] "=&v"(o[s].xl[2]), [ld##s] "=&v"(o[s].xl[3]),            \
        [ha##s] "=&v"(o[s].xh[0]), [hb##s] "=&v"(o[s].xh[1]), [hc##s] "=&v"(o[s].xh[2]),            \
        [hd##s] "=&v"(o[s].xh[3]), [pa##s] "=&v"(o[s].xp[0]), [pb##s] "=&v"(o[s].xp[1]),            \
        [pc##s] "=&v"(o[s].xp[2]), [pd##s] "=&v"(o[s].xp[3])
#define MD_SB_INS(s)                                                                              \
    [th##s] "v"(a_h + s * kQKBlockBytes), [tq##s] "v"(a_q + s * kQKBlockBytes),                     \
        [rl##s] "v"(a_lo + s * lo_step), [rh##s] "v"(a_hi + s * hi_step), [rp##s] "v"(a_p + s * 896u)

// Every LDS operand of a unit (nsb superblocks), then one wait.
template <int NSB>
__device__ __forceinline__ void md_read_unit(MdSb (&o)[NSB], uint32_t a_h, uint32_t a_q, uint32_t a_lo,
                                             uint32_t lo_step, uint32_t a_hi, uint32_t hi_step, uint32_t a_p) {
    static_assert(16 * 4 * kRecDwords == 896 && 4 * 4 * kRecDwords == 224, "record strides");
    if constexpr (NSB == 1)
        asm volatile(MD_SB_READS(0) "s_waitcnt lgkmcnt(0)" : MD_SB_OUTS(0) : MD_SB_INS(0) : "memory");
    else if constexpr (NSB == 2)
        asm volatile(MD_SB_READS(0) MD_SB_READS(1) "s_waitcnt lgkmcnt(0)"
                     : MD_SB_OUTS(0), MD_SB_OUTS(1)
                     : MD_SB_INS(0), MD_SB_INS(1)
                     : "memory");
    else if constexpr (NSB == 3)
        asm volatile(MD_SB_READS(0) MD_SB_READS(1) MD_SB_READS(2) "s_waitcnt lgkmcnt(0)"
                     : MD_SB_OUTS(0), MD_SB_OUTS(1), MD_SB_OUTS(2)
                     : MD_SB_INS(0), MD_SB_INS(1), MD_SB_INS(2)
                     : "memory");
    else
        asm volatile(MD_SB_READS(0) MD_SB_READS(1) MD_SB_READS(2) MD_SB_READS(3) "s_waitcnt lgkmcnt(0)"
                     : MD_SB_OUTS(0), MD_SB_OUTS(1), MD_SB_OUTS(2), MD_SB_OUTS(3)
                     : MD_SB_INS(0), MD_SB_INS(1), MD_SB_INS(2), MD_SB_INS(3)
                     : "memory");
}
// Q5_K: the same reads of superblock s plus the lane's qh bytes (at the
// quant address of a Q4_K row; the quants 32 bytes later).
#define MD5_SB_READS(s)                                                                            \
    "ds_read_b128 %[hv" #s "], %[th" #s "]\n\t"                                                   \
    "ds_read_b64 %[qh" #s "], %[tq" #s "]\n\t"                                                    \
    "ds_read_b64 %[qa" #s "], %[tq" #s "] offset:32\n\t"                                          \
    "ds_read_b64 %[qb" #s "], %[tq" #s "] offset:64\n\t"                                          \
    "ds_read_b64 %[qc" #s "], %[tq" #s "] offset:96\n\t"                                          \
    "ds_read_b64 %[qd" #s "], %[tq" #s "] offset:128\n\t"                                         \
    "ds_read_b64 %[la" #s "], %[rl" #s "]\n\t"                                                    \
    "ds_read_b64 %[lb" #s "], %[rl" #s "] offset:224\n\t"                                         \
    "ds_read_b64 %[lc" #s "], %[rl" #s "] offset:448\n\t"                                         \
    "ds_read_b64 %[ld" #s "], %[rl" #s "] offset:672\n\t"                                         \
    "ds_read_b64 %[ha" #s "], %[rh" #s "]\n\t"                                                    \
    "ds_read_b64 %[hb" #s "], %[rh" #s "] offset:224\n\t"                                         \
    "ds_read_b64 %[hc" #s "], %[rh" #s "] offset:448\n\t"                                         \
    "ds_read_b64 %[hd" #s "], %[rh" #s "] offset:672\n\t"                                         \
    "ds_read_b64 %[pa" #s "], %[rp" #s "]\n\t"                                                    \
    "ds_read_b64 %[pb" #s "], %[rp" #s "] offset:224\n\t"                                         \
    "ds_read_b64 %[pc" #s "], %[rp" #s "] offset:448\n\t"                                         \
    "ds_read_b64 %[pd" #s "], %[rp" #s "] offset:672\n\t"
#define MD5_SB_OUTS(s)                                                                             \
    [hv##s] "=&v"(o[s].hv), [qa##s] "=&v"(o[s].qb[0]), [qb##s] "=&v"(o[s].qb[1]),                  \
        [qc##s] "=&v"(o[s].qb[2]), [qd##s] "=&v"(o[s].qb[3]), [la##s] "=&v"(o[s].xl[0]),            \
        [lb##s] "=&v"(o[s].xl[1]), [lc##s] "=&v"(o[s].xl[2]), [ld##s] "=&v"(o[s].xl[3]),            \
        [ha##s] "=&v"(o[s].xh[0]), [hb##s] "=&v"(o[s].xh[1]), [hc##s] "=&v"(o[s].xh[2]),            \
        [hd##s] "=&v"(o[s].xh[3]), [pa##s] "=&v"(o[s].xp[0]), [pb##s] "=&v"(o[s].xp[1]),            \
        [pc##s] "=&v"(o[s].xp[2]), [pd##s] "=&v"(o[s].xp[3]), [qh##s] "=&v"(o[s].qh)
#define MD5_SB_INS(s)                                                                              \
    [th##s] "v"(a_h + s * kQ5KBlockBytes), [tq##s] "v"(a_q + s * kQ5KBlockBytes),                     \
        [rl##s] "v"(a_lo + s * lo_step), [rh##s] "v"(a_hi + s * hi_step), [rp##s] "v"(a_p + s * 896u)

// Every LDS operand of a Q5_K unit, then one wait.
template <int NSB>
__device__ __forceinline__ void md_read_unit5(MdSb (&o)[NSB], uint32_t a_h, uint32_t a_q, uint32_t a_lo,
                                             uint32_t lo_step, uint32_t a_hi, uint32_t hi_step, uint32_t a_p) {
    static_assert(16 * 4 * kRecDwords == 896 && 4 * 4 * kRecDwords == 224, "record strides");
    if constexpr (NSB == 1)
        asm volatile(MD5_SB_READS(0) "s_waitcnt lgkmcnt(0)" : MD5_SB_OUTS(0) : MD5_SB_INS(0) : "memory");
    else if constexpr (NSB == 2)
        asm volatile(MD5_SB_READS(0) MD5_SB_READS(1) "s_waitcnt lgkmcnt(0)"
                     : MD5_SB_OUTS(0), MD5_SB_OUTS(1)
                     : MD5_SB_INS(0), MD5_SB_INS(1)
                     : "memory");
    else if constexpr (NSB == 3)
        asm volatile(MD5_SB_READS(0) MD5_SB_READS(1) MD5_SB_READS(2) "s_waitcnt lgkmcnt(0)"
                     : MD5_SB_OUTS(0), MD5_SB_OUTS(1), MD5_SB_OUTS(2)
                     : MD5_SB_INS(0), MD5_SB_INS(1), MD5_SB_INS(2)
                     : "memory");
    else
        asm volatile(MD5_SB_READS(0) MD5_SB_READS(1) MD5_SB_READS(2) MD5_SB_READS(3) "s_waitcnt lgkmcnt(0)"
                     : MD5_SB_OUTS(0), MD5_SB_OUTS(1), MD5_SB_OUTS(2), MD5_SB_OUTS(3)
                     : MD5_SB_INS(0), MD5_SB_INS(1), MD5_SB_INS(2), MD5_SB_INS(3)
                     : "memory");
}
#undef MD_SB_READS
#undef MD_SB_OUTS
#undef MD_SB_INS
#undef MD5_SB_READS
#undef MD5_SB_OUTS
#undef MD5_SB_INS

// Lane 0 takes the next index from an LDS counter for the wave.
__device__ __forceinline__ int wave_grab(int *counter) {
    int v = 0;
    if ((threadIdx.x & 63) == 0) v = atomicAdd(counter, 1);
    return __builtin_amdgcn_readfirstlane(v);
}

struct MoeDownGeom {
    uint32_t wave_bytes;         // LDS per wave
    int tg;                      // tokens per workgroup
    uint32_t w_bytes, h_bytes;   // ranges: stacked down weights; h records
};

// DT: the down rows' type (Q4_K, Q5_K or Q6_K).
template <int NSB, int DT>
__global__ __launch_bounds__(kMdMaxWaves * 64) void moe_down_combine_kernel(
    const uint8_t *__restrict__ down, MoeDownGeom G, const uint8_t *__restrict__ hrec,
    const int32_t *__restrict__ ids, const float *__restrict__ wts, int T, int top_k, int H, int E,
    float *__restrict__ out) {
    constexpr bool Q6 = DT == kQ6_K, Q5 = DT == kQ5_K;
    constexpr uint32_t kRowBytes = md_row_bytes(NSB, DT), kPitch = md_pitch(NSB, DT);
    constexpr uint32_t kRecBytes = md_route_bytes(NSB);  // one route's records
    constexpr int kTF = md_full(md_tile_bytes(NSB, DT)), kTT = md_tail(md_tile_bytes(NSB, DT));
    constexpr int kRF = md_full(md_route_bytes(NSB)), kRT = md_tail(md_route_bytes(NSB));
    constexpr int kUnitLoads = kTF + kTT + kRF + kRT;  // every unit issues exactly this many
    constexpr uint32_t kTileSlot = md_slot(md_tile_bytes(NSB, DT)), kRouteSlot = md_slot(md_route_bytes(NSB));
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];  // sink, then waves x wave_bytes
    __shared__ float ys[kMdRoutes][16];
    __shared__ float rw[kMdRoutes];
    __shared__ int rok[kMdRoutes];
    __shared__ int it_e[kMdRoutes];
    __shared__ unsigned long long it_mask[kMdRoutes];
    __shared__ int n_items, next_item;

    const int lane = threadIdx.x & 63;
    const int wv = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
    const int row0 = (int)blockIdx.x * 16;
    const int t0 = (int)blockIdx.y * G.tg;
    const int nt = min(G.tg, T - t0);
    const int p0 = t0 * top_k;

    // Routing: route slot j = route p0 + j; an item is an expert with the
    // mask of its route slots.
    if (wv == 0) {
        int key = -1;
        float w = 0.0f;
        if (lane < nt * top_k) {
            const int e = ids[p0 + lane];
            w = wts[p0 + lane];
            if (e >= 0 && e < E && w != 0.0f) key = e;
        }
        rw[lane] = w;
        rok[lane] = key >= 0 ? 1 : 0;
        const uint64_t below = lane == 0 ? 0ull : (~0ull >> (64 - lane));
        int bits = 1;
        while ((1 << bits) <= E) bits++;
        const uint32_t k1 = (uint32_t)(key + 1);
        uint64_t same = __ballot(true);
        for (int bt = 0; bt < bits; bt++) {
            const uint64_t v = __ballot((k1 >> bt) & 1u);
            same &= ((k1 >> bt) & 1u) ? v : ~v;
        }
        const bool leader = key >= 0 && (same & below) == 0ull;
        const uint64_t lb = __ballot(leader);
        if (leader) {
            const int idx = __popcll(lb & below);
            it_e[idx] = key;
            it_mask[idx] = same;
        }
        if (lane == 0) {
            n_items = __popcll(lb);
            next_item = 0;
        }
    }
    if (threadIdx.x < 256) reinterpret_cast<uint32_t *>(lds)[threadIdx.x] = 0u;  // the sink
    __syncthreads();
    const int nitems = n_items;

    uint8_t *const sink = lds;  // always zero: reads of dead A lanes, writes of loads that move nothing
    uint8_t *const wbase = lds + 1024u + (uint32_t)wv * G.wave_bytes;
    const __amdgpu_buffer_rsrc_t rsw = wave_buffer(down, G.w_bytes);
    const __amdgpu_buffer_rsrc_t rsh = wave_buffer(hrec, G.h_bytes);
    const __amdgpu_buffer_rsrc_t rs0 = wave_buffer(hrec, 0);  // every load out of range
    // Per-lane offsets of the tile loads (row b / pitch, column b % pitch of
    // staged byte b: 1024 k + 16 lane for the full loads, then
    // 1024 kTF + 256 k + 4 lane for the tail) and of the record loads.
    uint32_t toff[kTF + kTT], roff[kRF + kRT];
#pragma unroll
    for (int k = 0; k < kTF + kTT; k++) {
        const uint32_t b = k < kTF ? 1024u * k + 16u * lane : 1024u * kTF + 256u * (k - kTF) + 4u * lane;
        const uint32_t r = b / kPitch, col = b - r * kPitch;
        toff[k] = (r < 16u && col < kRowBytes) ? r * kRowBytes + col : kMaskedOffset;
    }
#pragma unroll
    for (int k = 0; k < kRF + kRT; k++) {
        const uint32_t o = k < kRF ? 1024u * k + 16u * lane : 1024u * kRF + 256u * (k - kRF) + 4u * lane;
        roff[k] = o < kRecBytes ? o : kMaskedOffset;
    }
    auto mask_of = [&](int item) -> uint64_t {
        if (item >= nitems) return 0ull;
        const uint64_t m = it_mask[item];
        return ((uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)(m >> 32)) << 32) |
               (uint64_t)(uint32_t)__builtin_amdgcn_readfirstlane((int)(uint32_t)m);
    };
    // Items go to the waves as they ask (a wave sharing its SIMD takes fewer).
    auto grab = [&]() -> int { return wave_grab(&next_item); };
    // Issue cursor: the item whose units go out next and its routes left.
    int ii = grab();
    uint64_t im = mask_of(ii);
    bool ifirst = true;
    int its = kMdSlots - 1, irs = 0;  // last tile slot used; next route slot
    // Issues the next unit's loads (exactly kUnitLoads, all out of range when
    // no unit is left) and returns it as j | tile slot << 8 | route slot << 12,
    // or -1.
    auto issue_next = [&]() -> int {
        const bool have = __builtin_amdgcn_readfirstlane(ii < nitems ? 1 : 0) != 0;
        const bool tile = __builtin_amdgcn_readfirstlane(have && ifirst ? 1 : 0) != 0;
        if (tile) its = its == kMdSlots - 1 ? 0 : its + 1;
        const int e = have ? __builtin_amdgcn_readfirstlane(it_e[ii]) : 0;
        const uint32_t base = ((uint32_t)e * (uint32_t)H + (uint32_t)row0) * kRowBytes;
        // (one descriptor per branch: a selected one would be taken for divergent)
        // (Offsets go through named locals: an array element written in the
        // builtin's argument list breaks the kernel's host stub.)
        if (tile) {
            uint8_t *tdst = wbase + (uint32_t)its * kTileSlot;
#pragma unroll
            for (int k = 0; k < kTF; k++) {
                const uint32_t o = toff[k] + base;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_ptr)(tdst + 1024 * k), 16, o, 0, 0, kStreamLoad);
            }
#pragma unroll
            for (int k = kTF; k < kTF + kTT; k++) {
                const uint32_t o = toff[k] + base;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsw, (lds_ptr)(tdst + 1024 * kTF + 256 * (k - kTF)), 4, o, 0,
                                                         0, kStreamLoad);
            }
        } else {
#pragma unroll
            for (int k = 0; k < kTF; k++) {
                const uint32_t o = toff[k];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs0, (lds_ptr)sink, 16, o, 0, 0, 0);
            }
#pragma unroll
            for (int k = kTF; k < kTF + kTT; k++) {
                const uint32_t o = toff[k];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs0, (lds_ptr)sink, 4, o, 0, 0, 0);
            }
        }
        const int j = have ? __builtin_ctzll(im) : 0;
        const uint32_t rb = (uint32_t)(p0 + j) * kRecBytes;
        if (have) {
            uint8_t *rdst = wbase + kMdSlots * kTileSlot + (uint32_t)irs * kRouteSlot;
#pragma unroll
            for (int k = 0; k < kRF; k++) {
                const uint32_t o = roff[k] + rb;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsh, (lds_ptr)(rdst + 1024 * k), 16, o, 0, 0, 0);
            }
#pragma unroll
            for (int k = kRF; k < kRF + kRT; k++) {
                const uint32_t o = roff[k] + rb;
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rsh, (lds_ptr)(rdst + 1024 * kRF + 256 * (k - kRF)), 4, o, 0,
                                                         0, 0);
            }
        } else {
#pragma unroll
            for (int k = 0; k < kRF; k++) {
                const uint32_t o = roff[k];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs0, (lds_ptr)sink, 16, o, 0, 0, 0);
            }
#pragma unroll
            for (int k = kRF; k < kRF + kRT; k++) {
                const uint32_t o = roff[k];
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rs0, (lds_ptr)sink, 4, o, 0, 0, 0);
            }
        }
        const int unit = have ? (j | its << 8 | irs << 12) : -1;
        irs = irs == kMdSlots - 1 ? 0 : irs + 1;
        if (have) {
            im &= im - 1;
            ifirst = im == 0ull;
            if (ifirst) {
                ii = grab();
                im = mask_of(ii);
            }
        }
        return unit;
    };

    const int n = lane & 15, g = lane >> 4, q = n >> 2, pl = n & 3;
    const bool live = (g >> 1) == (q & 1) && pl < 3;
    const int hs = g >> 1;  // sub-block parity of this output lane's quarter
    const i32x4 zero4 = {0, 0, 0, 0};
    const uint32_t zero_lds = (uint32_t)(uintptr_t)(lds_ptr)sink;
    // A bytes 0..7 (q < 2) or 8..15 come from the records; the other half,
    // and every byte of a dead lane, from the zero sink.
    const bool lo_live = live && q < 2, hi_live = live && q >= 2;
    // y of the unit's route from its tile slot and route slot.
    auto compute = [&](int unit) {
        const int j = unit & 255, ts = (unit >> 8) & 15, rs = unit >> 12;
        const uint32_t tb = (uint32_t)(uintptr_t)(lds_ptr)(wbase + (uint32_t)ts * kTileSlot);
        const uint32_t rb = (uint32_t)(uintptr_t)(lds_ptr)(wbase + kMdSlots * kTileSlot + (uint32_t)rs * kRouteSlot);
        const uint32_t a_h0 = tb + n * kPitch, a_q0 = a_h0 + 16 + 8 * g;
        // records of groups 16 s + 4 c + q (A) and 16 s + 4 c + g (scale, sum)
        const uint32_t a_x = rb + 4 * kRecDwords * q + 16 * (pl < 3 ? pl : 0) + 8 * (g & 1);
        const uint32_t a_lo0 = lo_live ? a_x : zero_lds, a_hi0 = hi_live ? a_x : zero_lds;
        const uint32_t lo_step = lo_live ? 16u * 4 * kRecDwords : 0u, hi_step = hi_live ? 16u * 4 * kRecDwords : 0u;
        const uint32_t a_p0 = rb + 4 * kRecDwords * g + 48;
        MdSb o[NSB];
        if constexpr (Q5)
            md_read_unit5<NSB>(o, a_h0, a_q0, a_lo0, lo_step, a_hi0, hi_step, a_p0);
        else
            md_read_unit<NSB>(o, a_h0, a_q0, a_lo0, lo_step, a_hi0, hi_step, a_p0);
        // every superblock's products first, then their epilogues
        i32x4 Dall[NSB][4];
#pragma unroll
        for (int s = 0; s < NSB; s++)
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint2 qv = o[s].qb[c];
                uint32_t b0 = qv.x & 0x0F0F0F0Fu, b1 = qv.y & 0x0F0F0F0Fu;
                uint32_t b2 = (qv.x >> 4) & 0x0F0F0F0Fu, b3 = (qv.y >> 4) & 0x0F0F0F0Fu;
                if constexpr (Q5) {  // fifth bits: bit 2 c (low nibbles), 2 c + 1 (high) of qh
                    const uint2 hq = o[s].qh;
                    b0 |= ((hq.x >> (2 * c)) & 0x01010101u) << 4;
                    b1 |= ((hq.y >> (2 * c)) & 0x01010101u) << 4;
                    b2 |= ((hq.x >> (2 * c + 1)) & 0x01010101u) << 4;
                    b3 |= ((hq.y >> (2 * c + 1)) & 0x01010101u) << 4;
                }
                const i32x4 B = {(int)b0, (int)b1, (int)b2, (int)b3};
                const i32x4 A = {(int)o[s].xl[c].x, (int)o[s].xl[c].y, (int)o[s].xh[c].x, (int)o[s].xh[c].y};
                Dall[s][c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, zero4, 0, 0, 0);
            }
        float v = 0.0f;
#pragma unroll
        for (int s = 0; s < NSB; s++) {
            const u32x4 hv = o[s].hv;
            const float2 *xp = o[s].xp;
            const i32x4 *D = Dall[s];
            const float d = half_bits_to_float_fast(hv.x);
            const float dmin = half_bits_to_float_fast(hv.x >> 16);
            // 6-bit codes (RT/GgufKQuantLayout.java:37-49) of sub-blocks hs, 2 + hs, 4 + hs, 6 + hs
            const uint32_t hy = hv.y >> (8 * hs), hz = hv.z >> (8 * hs), hw = hv.w >> (8 * hs);
            const uint32_t sc03 = hy & 0x003F003Fu;
            const uint32_t mn03 = hz & 0x003F003Fu;
            const uint32_t sc47 = (hw & 0x000F000Fu) | ((hy >> 2) & 0x00300030u);
            const uint32_t mn47 = ((hw >> 4) & 0x000F000Fu) | ((hz >> 2) & 0x00300030u);
            const float scf[4] = {(float)(sc03 & 0xFFu), (float)((sc03 >> 16) & 0xFFu),
                                  (float)(sc47 & 0xFFu), (float)((sc47 >> 16) & 0xFFu)};
            const float mnf[4] = {(float)(mn03 & 0xFFu), (float)((mn03 >> 16) & 0xFFu),
                                  (float)(mn47 & 0xFFu), (float)((mn47 >> 16) & 0xFFu)};
            float S[4];
#pragma unroll
            for (int c = 0; c < 4; c++)
                S[c] = (float)(int)(((uint32_t)D[c][2] << 16) + (((uint32_t)D[c][1] << 8) + (uint32_t)D[c][0])) *
                       xp[c].x;
            if (__builtin_isfinite(d) && __builtin_isfinite(dmin)) {
                float qs = 0.0f, mm = 0.0f;
#pragma unroll
                for (int c = 0; c < 4; c++) {
                    qs = fmaf(scf[c], S[c], qs);
                    mm = fmaf(mnf[c], xp[c].y, mm);
                }
                v += fmaf(d, qs, -(dmin * mm));
            } else {
                // the reference's (d sc) products; zero min codes skip a
                // non-finite dmin (minContribution, RT/GgufKQuantLayout.java:67-69)
#pragma unroll
                for (int c = 0; c < 4; c++)
                    v += (d * scf[c]) * S[c] - (mnf[c] != 0.0f ? dmin * mnf[c] : 0.0f) * xp[c].y;
            }
        }
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (lane < 16) lds_store_f32((uint32_t)(uintptr_t)(lds_ptr)&ys[j][lane], v);
    };

    // Q6_K down rows: chunk c of a superblock (half c >> 1, part c & 1)
    // covers elements 128 (c >> 1) + 32 (c & 1) + l and + 64 (l < 32), so A
    // row 4 q + p reads record group 8 (c >> 1) + 2 (c & 1) + 4 (q >> 1) +
    // (q & 1) (16 elements: the second run for q >= 2, half q & 1), and the
    // quarter's scale is byte 8 (c >> 1) + 2 (c & 1) + 4 (g >> 1) + (g & 1)
    // of the superblock's int8 scales.  Rows are 210 s + 16-row-aligned
    // bytes apart, so a lane's superblock starts 0 or 2 bytes off a dword:
    // it reads aligned dwords and realigns them (v_alignbyte_b32).  The -32
    // offset enters as -32 times the quarter's fp32 sum of h.
    auto compute_q6 = [&](int unit) {
        const int j = unit & 255, ts = (unit >> 8) & 15, rs = unit >> 12;
        const uint32_t tb = (uint32_t)(uintptr_t)(lds_ptr)(wbase + (uint32_t)ts * kTileSlot);
        const uint32_t rb = (uint32_t)(uintptr_t)(lds_ptr)(wbase + kMdSlots * kTileSlot + (uint32_t)rs * kRouteSlot);
        const uint32_t a_x = rb + 4 * kRecDwords * (4 * (q >> 1) + (q & 1)) + 16 * (pl < 3 ? pl : 0) + 8 * (g & 1);
        const uint32_t a_lo0 = lo_live ? a_x : zero_lds, a_hi0 = hi_live ? a_x : zero_lds;
        const uint32_t lo_step = lo_live ? 16u * 4 * kRecDwords : 0u, hi_step = hi_live ? 16u * 4 * kRecDwords : 0u;
        const uint32_t a_p0 = rb + 4 * kRecDwords * (4 * hs + (g & 1)) + 48;
        float v = 0.0f;
#pragma unroll
        for (int s = 0; s < NSB; s++) {
            const uint32_t sa = tb + (uint32_t)n * kRowBytes + (uint32_t)s * kQ6KBlockBytes;
            const uint32_t sh = sa & 3u, ab = sa - sh, aq = ab + 8u * (uint32_t)g;
            uint2 p01[6], s01, s23, xl[4], xh[4];
            uint32_t p2[6], s4;
            float2 xp[4];
            static_assert(4 * kRecDwords * 2 == 112 && 4 * kRecDwords * 8 == 448 && 4 * kRecDwords * 10 == 560,
                          "record offsets of chunks 1..3");
            asm volatile(
                "ds_read2_b32 %0, %27 offset1:1\n\t"
                "ds_read_b32 %6, %27 offset:8\n\t"
                "ds_read2_b32 %1, %27 offset0:8 offset1:9\n\t"
                "ds_read_b32 %7, %27 offset:40\n\t"
                "ds_read2_b32 %2, %27 offset0:16 offset1:17\n\t"
                "ds_read_b32 %8, %27 offset:72\n\t"
                "ds_read2_b32 %3, %27 offset0:24 offset1:25\n\t"
                "ds_read_b32 %9, %27 offset:104\n\t"
                "ds_read2_b32 %4, %27 offset0:32 offset1:33\n\t"
                "ds_read_b32 %10, %27 offset:136\n\t"
                "ds_read2_b32 %5, %27 offset0:40 offset1:41\n\t"
                "ds_read_b32 %11, %27 offset:168\n\t"
                "ds_read2_b32 %12, %28 offset0:48 offset1:49\n\t"
                "ds_read2_b32 %13, %28 offset0:50 offset1:51\n\t"
                "ds_read_b32 %14, %28 offset:208\n\t"
                "ds_read_b64 %15, %29\n\t"
                "ds_read_b64 %16, %29 offset:112\n\t"
                "ds_read_b64 %17, %29 offset:448\n\t"
                "ds_read_b64 %18, %29 offset:560\n\t"
                "ds_read_b64 %19, %30\n\t"
                "ds_read_b64 %20, %30 offset:112\n\t"
                "ds_read_b64 %21, %30 offset:448\n\t"
                "ds_read_b64 %22, %30 offset:560\n\t"
                "ds_read_b64 %23, %31\n\t"
                "ds_read_b64 %24, %31 offset:112\n\t"
                "ds_read_b64 %25, %31 offset:448\n\t"
                "ds_read_b64 %26, %31 offset:560\n\t"
                "s_waitcnt lgkmcnt(0)"
                : "=&v"(p01[0]), "=&v"(p01[1]), "=&v"(p01[2]), "=&v"(p01[3]), "=&v"(p01[4]), "=&v"(p01[5]),
                  "=&v"(p2[0]), "=&v"(p2[1]), "=&v"(p2[2]), "=&v"(p2[3]), "=&v"(p2[4]), "=&v"(p2[5]), "=&v"(s01),
                  "=&v"(s23), "=&v"(s4), "=&v"(xl[0]), "=&v"(xl[1]), "=&v"(xl[2]), "=&v"(xl[3]), "=&v"(xh[0]),
                  "=&v"(xh[1]), "=&v"(xh[2]), "=&v"(xh[3]), "=&v"(xp[0]), "=&v"(xp[1]), "=&v"(xp[2]), "=&v"(xp[3])
                : "v"(aq), "v"(ab), "v"(a_lo0 + s * lo_step), "v"(a_hi0 + s * hi_step),
                  "v"(a_p0 + 16u * 4 * kRecDwords * s)
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
                    b[k] = (ql[c][k] & 0x0F0F0F0Fu) | ((pt == 0 ? hq << 4 : hq << 2) & 0x30303030u);
                    b[2 + k] = ((ql[c][k] >> 4) & 0x0F0F0F0Fu) | ((pt == 0 ? hq : hq >> 2) & 0x30303030u);
                }
                const i32x4 B = {(int)b[0], (int)b[1], (int)b[2], (int)b[3]};
                const i32x4 A = {(int)xl[c].x, (int)xl[c].y, (int)xh[c].x, (int)xh[c].y};
                D[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A, B, zero4, 0, 0, 0);
            }
            const uint32_t slo = hs ? s1 : s0, shi = hs ? s3 : s2;
            float vs = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; c++) {
                const uint32_t sw = (c >> 1) ? shi : slo;
                const float scv = (float)(int)(int8_t)((sw >> (8 * ((g & 1) + 2 * (c & 1)))) & 0xFFu);
                // sum q X over the quarter can reach 16 * 63 * 2^22 > 2^31:
                // the planes combine in fp32 (relative error under 2^-23)
                const float S = fmaf((float)D[c][2], 65536.0f, (float)(D[c][0] + 256 * D[c][1]));
                vs = fmaf(scv, fmaf(S, xp[c].x, -32.0f * xp[c].y), vs);
            }
            v = fmaf(d, vs, v);
        }
        v += __shfl_xor(v, 16);
        v += __shfl_xor(v, 32);
        if (lane < 16) lds_store_f32((uint32_t)(uintptr_t)(lds_ptr)&ys[j][lane], v);
    };

    // Unit k's loads go out before unit k - (kMdSlots - 1) is computed.
    int u0 = issue_next(), u1 = kMdSlots > 2 ? issue_next() : -1;
    while (u0 >= 0) {  // uniform
        wait_vm<kUnitLoads * (kMdSlots - 2)>();  // unit u0's loads are done (later units' may not be)
        const int un = issue_next();
        if constexpr (Q6) compute_q6(u0);
        else compute(u0);
        if constexpr (kMdSlots > 2) {
            u0 = u1;
            u1 = un;
        } else {
            u0 = un;
        }
    }
    asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)" ::: "memory");
    __syncthreads();
    {
#pragma clang fp contract(off)
        for (int o = (int)threadIdx.x; o < nt * 16; o += (int)blockDim.x) {
            const int t = o >> 4, r = o & 15;
            float acc = 0.0f;
            for (int j = 0; j < top_k; j++) {
                const int slot = t * top_k + j;
                const float scaled = ys[slot][r] * rw[slot];  // AccelOps.mulScalar
                acc = rok[slot] ? acc + scaled : acc;         // addToTokenRow
            }
            out[(int64_t)(t0 + t) * H + row0 + r] = acc;
        }
    }
}

namespace {

// Bytes of a row's 256-column piece: a Q4_K superblock (144, as eight Q4_0
// blocks), a Q5_K superblock (176) or a Q6_K superblock (210).
constexpr uint32_t piece_bytes(int type) {
    return type == kQ6_K ? 210u : type == kQ5_K ? kQ5KBlockBytes : kQKBlockBytes;
}

// 1 KB loads an item slot holds for `type` rows.
int max_dma(int type) {
    return type == kQ6_K   ? MoRing<kQ6_K>::kMaxDma
           : type == kQ5_K ? MoRing<kQ5_K>::kMaxDma
           : type == kQ4_0 ? MoRing<kQ4_0>::kMaxDma
                           : MoRing<kQ4_K>::kMaxDma;
}

// Geometry of pass `mode` over `type` rows.  The caller has checked that H
// and I are multiples of 256 in [256, 4096].
MoeTileGeom make_geom(int mode, int E, int H, int I, int type) {
    const uint32_t pb = piece_bytes(type);
    const int kMoMaxDma = max_dma(type);
    MoeTileGeom g{};
    const int K = mode == 0 ? H : I;
    // a pitch whose 16-byte units are odd modulo 16 spreads 16 rows over all
    // banks (Q6_K rows, 210 bytes a superblock, rounded up to 16 bytes first)
    auto pitch_of = [pb](int nsb) {
        const uint32_t rb = ((uint32_t)nsb * pb + 15u) / 16u * 16u;
        return (rb / 16) % 2 == 1 ? rb : rb + 16;
    };
    auto part_dma_of = [&](int nsb, int rt) { return (16 * rt * (int)pitch_of(nsb) + 1023) / 1024; };
    // Gate/up items hold 16 rows of both matrices, one wave per superblock
    // and matrix (so at most 8 superblocks), both within a slot: longer rows
    // (an even count of superblocks) are cut in halves.
    g.halves = mode == 0 && (K / kQK > 8 || 2 * part_dma_of(K / kQK, 1) > kMoMaxDma) ? 2 : 1;
    g.nsb = K / kQK / g.halves;
    g.rows_e = mode == 0 ? I : H;
    // Down items: as many 16-row tiles as waves (one per tile and
    // superblock, at most 8 tiles) and a slot take.
    g.rt = mode == 0 ? 1 : min(16 / g.nsb, 8);
    while (g.rt > 1 && part_dma_of(g.nsb, g.rt) > kMoMaxDma) g.rt--;
    g.tiles_e = g.halves * ((g.rows_e + 16 * g.rt - 1) / (16 * g.rt));
    g.row_bytes = (uint32_t)g.nsb * pb;
    g.stride = (uint32_t)(g.halves * g.row_bytes);
    g.pitch = pitch_of(g.nsb);
    g.part_dma = part_dma_of(g.nsb, g.rt);
    g.ndma = mode == 0 ? 2 * g.part_dma : g.part_dma;
    g.vec_len = K;
    g.out_len = g.rows_e;
    g.w_bytes = (int64_t)E * g.rows_e * g.stride;
    return g;
}

// The token-major down pass: I up to 1024 (a wave's slots fit at least one
// wave), top_k <= 64 and 32-bit buffer offsets.
constexpr int kMdStaticLds = kMdRoutes * (16 * 4 + 4 + 4 + 4 + 8) + 16;  // ys, rw, rok, it_e, it_mask, counters
constexpr int kLdsBytes = 163840;

bool make_down_geom(int E, int H, int I, int T, int top_k, int dt, MoeDownGeom &g, int &waves) {
    const int nsb = I / kQK;
    if (nsb < 1 || nsb > 4 || top_k < 1 || top_k > kMdRoutes || H % 16 != 0) return false;
    g.wave_bytes = (uint32_t)(kMdSlots * (md_slot(md_tile_bytes(nsb, dt)) + md_slot(md_route_bytes(nsb))));
    g.tg = kMdRoutes / top_k;
    const int64_t w_bytes = (int64_t)E * H * md_row_bytes(nsb, dt);
    const int64_t h_bytes = (int64_t)T * top_k * (I / 16) * kRecDwords * 4;
    if (w_bytes >= (int64_t)kMaskedOffset || h_bytes >= (int64_t)kMaskedOffset) return false;
    g.w_bytes = (uint32_t)w_bytes;
    g.h_bytes = (uint32_t)h_bytes;
    waves = min(kMdMaxWaves, (int)((kLdsBytes - kMdStaticLds - 1024) / (int)g.wave_bytes));
    return waves >= 1;
}

// Shapes every tile pass takes: hidden and inter multiples of 256 up to
// 4096, the routing tables in LDS, x 16-byte aligned (nullptr: shape only).
bool tile_shape_ok(int E, int H, int I, int P, const float *x) {
    return H >= kQK && I >= kQK && H % kQK == 0 && I % kQK == 0 && H <= 16 * kQK && I <= 16 * kQK &&
           E <= kMoMaxExperts && P <= kMoMaxRoutes && (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
}

// Whether pass `mode` over `type` rows fits the kernel (after tile_shape_ok).
bool tile_pass_ok(int mode, int E, int H, int I, int type) {
    const MoeTileGeom g = make_geom(mode, E, H, I, type);
    if (g.halves == 2 && ((mode == 0 ? H : I) / kQK) % 2 != 0) return false;  // halves of equal length
    if ((mode == 0 ? 2 * g.nsb : g.rt * g.nsb) > kMoWaves) return false;
    return g.ndma <= max_dma(type) && g.w_bytes < (int64_t)kMaskedOffset && 2 * kMoGroup * 16 * g.rt <= kMoOutCap;
}

// The token-major down pass takes Q4_K, Q5_K and Q6_K rows where its
// geometry fits.  It reads an expert's down tile once per token group (64 /
// top_k tokens) that routes to it, the expert-major pass once per group of
// four of its routes: past kTokenMajorMaxGroups token groups (prefill) the
// expert-major pass moves fewer bytes and takes the Q4_K / Q5_K rows.
constexpr int kTokenMajorMaxGroups = 4;
bool token_major_down(int down_type, int E, int H, int I, int T, int top_k, MoeDownGeom &gd, int &waves) {
    if (down_type != kQ4_K && down_type != kQ5_K && down_type != kQ6_K) return false;
    if (!make_down_geom(E, H, I, T, top_k, down_type, gd, waves)) return false;
    return down_type == kQ6_K || (T + gd.tg - 1) / gd.tg <= kTokenMajorMaxGroups ||
           !tile_pass_ok(1, E, H, I, down_type);
}

}  // namespace

bool moe_kq_mfma_supported(int gate_type, int down_type, int E, int H, int I, int T, int top_k,
                           const float *x) {
    if (gate_type != kQ4_K && gate_type != kQ5_K && gate_type != kQ6_K) return false;
    if (!tile_shape_ok(E, H, I, T * top_k, x) || !tile_pass_ok(0, E, H, I, gate_type)) return false;
    // Q6_K gate / up: one half (hidden up to 2048) of rows that start on a
    // dword (an even superblock count), as the loads into the ring need
    if (gate_type == kQ6_K && (make_geom(0, E, H, I, kQ6_K).halves != 1 || (H / kQK) % 2 != 0)) return false;
    MoeDownGeom gd;
    int waves = 0;
    if (token_major_down(down_type, E, H, I, T, top_k, gd, waves)) return true;
    return (down_type == kQ4_K || down_type == kQ5_K) && tile_pass_ok(1, E, H, I, down_type);
}

bool moe_q40_mfma_supported(int E, int H, int I, int P, const float *x) {
    // gate / up rows in one half (hidden up to 2048)
    return H <= 8 * kQK && tile_shape_ok(E, H, I, P, x) && tile_pass_ok(0, E, H, I, kQ4_0) &&
           tile_pass_ok(1, E, H, I, kQ4_0);
}

// Gate/up then down: with the token-major down pass two launches, h as
// digit records; otherwise gate/up, the expert-major down pass and the
// combine.  Each pass routes in LDS first.  The caller has checked
// moe_kq_mfma_supported.
hipError_t launch_moe_kq_mfma(int gate_type, int down_type, const uint8_t *gate, const uint8_t *up,
                              const uint8_t *down, int E, int H, int I, const float *x, const int32_t *ids,
                              const float *wts, int T, int top_k, float *out, uint8_t *ws, hipStream_t stream) {
    const MoeLayout L = moe_layout(T, top_k, H, I, E);
    const int P = T * top_k;
    const MoeTileGeom g0 = make_geom(0, E, H, I, gate_type);
    const unsigned grid = (unsigned)device_cus();
    float *hbuf = reinterpret_cast<float *>(ws + L.h);
    // h records (P I 3.5 bytes) fit the fp32 h region.
    MoeDownGeom gd;
    int waves = 0;
    const bool rec = token_major_down(down_type, E, H, I, T, top_k, gd, waves);
    if (!rec && down_type != kQ4_K && down_type != kQ5_K) return hipErrorNotSupported;
    auto gate_up = [&](auto kernel) {
        hipLaunchKernelGGL(kernel, dim3(grid), dim3(kMoThreads), 0, stream, gate, up, g0, x, top_k, ids, wts, E, P,
                           hbuf);
    };
    switch ((gate_type == kQ6_K ? 8 : gate_type == kQ5_K ? 4 : 0) + (rec ? 2 : 0) + (g0.halves == 2 ? 1 : 0)) {
    case 8: gate_up(&moe_expert_tile_kernel<0, false, 1, kQ6_K>); break;
    case 10: gate_up(&moe_expert_tile_kernel<0, true, 1, kQ6_K>); break;
    case 0: gate_up(&moe_expert_tile_kernel<0, false, 1, kQ4_K>); break;
    case 1: gate_up(&moe_expert_tile_kernel<0, false, 2, kQ4_K>); break;
    case 2: gate_up(&moe_expert_tile_kernel<0, true, 1, kQ4_K>); break;
    case 3: gate_up(&moe_expert_tile_kernel<0, true, 2, kQ4_K>); break;
    case 4: gate_up(&moe_expert_tile_kernel<0, false, 1, kQ5_K>); break;
    case 5: gate_up(&moe_expert_tile_kernel<0, false, 2, kQ5_K>); break;
    case 6: gate_up(&moe_expert_tile_kernel<0, true, 1, kQ5_K>); break;
    case 7: gate_up(&moe_expert_tile_kernel<0, true, 2, kQ5_K>); break;
    default: return hipErrorNotSupported;  // Q6_K in halves: moe_kq_mfma_supported refuses it
    }
    if (rec) {
        const dim3 dgrid((unsigned)(H / 16), (unsigned)((T + gd.tg - 1) / gd.tg));
        const size_t lds = 1024 + (size_t)waves * gd.wave_bytes;
        const uint8_t *hrec = ws + L.h;
        auto run = [&](auto kernel) {
            if (lds > 65536) {
                const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(kernel),
                                                         hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
                if (e != hipSuccess) return e;
            }
            hipLaunchKernelGGL(kernel, dgrid, dim3(64 * waves), lds, stream, down, gd, hrec, ids, wts, T, top_k,
                               H, E, out);
            return hipGetLastError();
        };
        switch (I / kQK + (down_type == kQ6_K ? 4 : down_type == kQ5_K ? 8 : 0)) {
        case 1: return run(&moe_down_combine_kernel<1, kQ4_K>);
        case 2: return run(&moe_down_combine_kernel<2, kQ4_K>);
        case 3: return run(&moe_down_combine_kernel<3, kQ4_K>);
        case 4: return run(&moe_down_combine_kernel<4, kQ4_K>);
        case 5: return run(&moe_down_combine_kernel<1, kQ6_K>);
        case 6: return run(&moe_down_combine_kernel<2, kQ6_K>);
        case 7: return run(&moe_down_combine_kernel<3, kQ6_K>);
        case 8: return run(&moe_down_combine_kernel<4, kQ6_K>);
        case 9: return run(&moe_down_combine_kernel<1, kQ5_K>);
        case 10: return run(&moe_down_combine_kernel<2, kQ5_K>);
        case 11: return run(&moe_down_combine_kernel<3, kQ5_K>);
        default: return run(&moe_down_combine_kernel<4, kQ5_K>);
        }
    }
    float *ypair = reinterpret_cast<float *>(ws + L.ypair);
    const MoeTileGeom g1 = make_geom(1, E, H, I, down_type);
    if (down_type == kQ5_K)
        hipLaunchKernelGGL((moe_expert_tile_kernel<1, false, 1, kQ5_K>), dim3(grid), dim3(kMoThreads), 0, stream,
                           down, (const uint8_t *)nullptr, g1, (const float *)hbuf, top_k, ids, wts, E, P, ypair);
    else
        hipLaunchKernelGGL((moe_expert_tile_kernel<1, false, 1, kQ4_K>), dim3(grid), dim3(kMoThreads), 0, stream,
                           down, (const uint8_t *)nullptr, g1, (const float *)hbuf, top_k, ids, wts, E, P, ypair);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_moe_combine(ids, wts, ypair, T, top_k, H, E, out, stream);
}

// All-Q4_0 experts: gate/up (fp32 h), the expert-major down pass and the
// combine, the Q4_K kernels' passes with Q4_0's contraction.  The caller has
// checked moe_q40_mfma_supported.
hipError_t launch_moe_q40_mfma(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int E, int H, int I,
                               const float *x, const int32_t *ids, const float *wts, int T, int top_k, float *out,
                               uint8_t *ws, hipStream_t stream) {
    const MoeLayout L = moe_layout(T, top_k, H, I, E);
    const int P = T * top_k;
    const MoeTileGeom g0 = make_geom(0, E, H, I, kQ4_0), g1 = make_geom(1, E, H, I, kQ4_0);
    const unsigned grid = (unsigned)device_cus();
    float *hbuf = reinterpret_cast<float *>(ws + L.h);
    float *ypair = reinterpret_cast<float *>(ws + L.ypair);
    hipLaunchKernelGGL((moe_expert_tile_kernel<0, false, 1, kQ4_0>), dim3(grid), dim3(kMoThreads), 0, stream, gate,
                       up, g0, x, top_k, ids, wts, E, P, hbuf);
    hipLaunchKernelGGL((moe_expert_tile_kernel<1, false, 1, kQ4_0>), dim3(grid), dim3(kMoThreads), 0, stream, down,
                       (const uint8_t *)nullptr, g1, (const float *)hbuf, top_k, ids, wts, E, P, ypair);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_moe_combine(ids, wts, ypair, T, top_k, H, E, out, stream);
}

}  // namespace gollek
