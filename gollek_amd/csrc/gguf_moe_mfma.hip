// gguf_moe_mfma.hip -- grouped Q4_K MoE expert FFN on the gfx950 matrix cores.
//
// Semantics as gguf_moe.hip (MoeForwardPass.java:217-240, :461-472; swigluFfn
// DirectForwardFfnService.java:40-61): h_pair = silu(gate_e x_t) * (up_e x_t),
// y_pair = down_e h_pair, out[t] = sum_j w[t,j] y_pair[t,j] in route order.
//
// Two passes of one tile kernel, after the routing kernel has sorted the
// valid routes by expert and laid out work items:
//   pass 0 (gate/up): item = (used expert, 16-row tile of its I rows, group of
//     up to 4 of its routes).  A slot holds the tile's 16 gate rows and 16 up
//     rows; wave w < nsb contracts gate superblock w, wave nsb + w up
//     superblock w; h = silu(g) u per route and row.
//   pass 1 (down): item = (used expert, RT = 16 / nsb 16-row tiles of its H
//     rows, route group); wave w = (row tile w / nsb, superblock w % nsb).
// The Q4_K contraction is the one of gguf_gemv_mfma.hip's kernels
// (v_mfma_i32_16x16x64_i8 over balanced 22-bit digits of the vector, low and
// high nibbles as bytes 0..15), with two routes per MFMA: A rows 8 t + 4 h + p hold route t's digits, so its
// results sit in output lanes 32 t + 16 h + n and the second route costs no
// extra epilogue instructions.
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
// ring waits on.
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
constexpr int kMoMaxDma = 38;        // 1 KB loads per item slot
constexpr int kMoDmaPerWave = (kMoMaxDma + kMoWaves - 1) / kMoWaves;
constexpr int kMoSlot = kMoMaxDma * 1024;
constexpr int kMoSlots = 3;
constexpr int kMoOutCap = 2560;      // buffered results (value, index)

}  // namespace

// Host-computed geometry of one pass.
struct MoeTileGeom {
    int nsb;          // superblocks per weight row (K / 256)
    int rows_e;       // weight rows per expert
    int rt;           // 16-row tiles per item (pass 0: 1)
    int tiles_e;      // items per expert and route group
    uint32_t row_bytes, pitch;
    int part_dma;     // loads per matrix part (pass 0) or per item (pass 1)
    int ndma;         // loads per item
    int vec_len;      // vector length (K)
    int out_len;      // result length per route (rows per expert)
    int64_t w_bytes;  // bytes of one stacked weight matrix (< 2^31)
};

// MODE 0: gate/up (w0 = gate, w1 = up); MODE 1: down (w0 = down).
// vec: pass 0 x[T][H] (route p -> token p / top_k); pass 1 h[P][I] (route p).
template <int MODE>
__global__ __launch_bounds__(kMoThreads) void moe_expert_tile_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, MoeTileGeom G,
    const float *__restrict__ vec, int top_k, const int32_t *__restrict__ meta, int E, int P,
    float *__restrict__ out) {
    __shared__ __attribute__((aligned(16))) uint8_t ring[kMoSlots * kMoSlot + 1024];  // + sink
    __shared__ __attribute__((aligned(16))) uint8_t scratch[kMoWaves][1024];  // digit build
    __shared__ float part[2][kMoGroup][kMoWaves][16];
    __shared__ float outv[kMoOutCap];
    __shared__ int outi[kMoOutCap];
    __shared__ int gid[kMoGroup];  // route ids of the current group

    const int32_t *counts = meta, *offsets = meta + E, *pairs = meta + 2 * E + 1;
    const int32_t *used = pairs + P;
    const int nused = used[E];
    const int32_t *items = used + E + 1 + (MODE == 1 ? E + 1 : 0);
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
    if (unit_split) {
        const int unit = (int)blockIdx.x / kpu, sub = (int)blockIdx.x - unit * kpu;
        i_begin = unit < nunits ? unit * G.tiles_e + sub * G.tiles_e / kpu : 0;
        i_end = unit < nunits ? unit * G.tiles_e + (sub + 1) * G.tiles_e / kpu : 0;
    } else {
        i_begin = (int)((int64_t)blockIdx.x * nitems / gridDim.x);
        i_end = (int)((int64_t)(blockIdx.x + 1) * nitems / gridDim.x);
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
        int u, e, group, tile, ntok, row0, nrows;
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
        c.cnt = counts[c.e];
        c.groups = (c.cnt + kMoGroup - 1) / kMoGroup;
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
            c.cnt = counts[c.e];
            c.groups = (c.cnt + kMoGroup - 1) / kMoGroup;
        }
    };
    auto item_of = [&](const Cursor &c) {
        Item it;
        it.u = c.u;
        it.e = c.e;
        it.group = c.group;
        it.tile = c.tile;
        it.ntok = min(kMoGroup, c.cnt - kMoGroup * c.group);
        it.row0 = c.tile * rows_item;
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
            base = (uint32_t)(((int64_t)it.e * G.rows_e + it.row0) * G.row_bytes);
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
                                                     ok ? base + r * G.row_bytes + col : kMaskedOffset,
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
    const uint32_t a_h0 = ring_base + mat * part_off + (rtile * 16 + n) * G.pitch + sb * kQKBlockBytes;
    const uint32_t a_q0 = a_h0 + 16 + 8 * g;
    const i32x4 zero4 = {0, 0, 0, 0};

    // Operands of the current route group: A per MFMA pair and chunk; per
    // output lane the sub-block sums and the superblock scale of its route.
    i32x4 A[2][4];
    float xs4[2][4], xs[2];
    int cur_key = -1;  // e * 65536 + group of the operands held

    // Digits of route group `it` for this wave's superblock.
    // `between` runs after the vector loads are issued and before they are
    // used: in the prologue it issues the first items' loads, so the wait for
    // the vectors (issued first) does not wait for those.  Mid-stream
    // (drain = true) the vectors queue behind the ring's loads anyway.
    auto build = [&](const Item &it, bool drain, auto &&between) {
#pragma unroll
        for (int pp = 0; pp < 2; pp++)
#pragma unroll
            for (int c = 0; c < 4; c++) {
                A[pp][c] = i32x4{0, 0, 0, 0};
                xs4[pp][c] = 0.0f;
            }
        xs[0] = xs[1] = 0.0f;
        if (!active) {
            between();
            return;
        }
        const uint32_t sbase = (uint32_t)(uintptr_t)(lds_ptr)scratch[wv];
        float4 v[kMoGroup];
        // loads first, then one wait (this also drains the ring's loads)
#pragma unroll
        for (int j = 0; j < kMoGroup; j++) {
            const int p = pairs[offsets[it.e] + kMoGroup * it.group + min(j, it.ntok - 1)];
            if (wv == 0 && lane == 0) gid[j] = p;  // route ids for the reductions
            const int vi = MODE == 0 ? p / top_k : p;
            v[j] = reinterpret_cast<const float4 *>(vec + (int64_t)vi * G.vec_len + sb * kQK)[lane];
        }
        between();
        if (drain) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        // Consume every loaded vector so the compiler's own wait comes here
        // (it cannot see the one above): a load it still thought outstanding
        // would make it wait for all loads before the next write of its registers.
        asm volatile("" ::"v"(v[0].x), "v"(v[1].x), "v"(v[2].x), "v"(v[3].x));
#pragma unroll
        for (int j = 0; j < kMoGroup; j++) {
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
            sx = sum8_i(sx);
            const float scale = finite ? ldexpf(1.0f, ex - 22) : __builtin_nanf("");
            // scratch: planes at 0 / 256 / 512, sub-block sums (fp32) at 768 + 4 j,
            // scale at 832
            asm volatile(
                "ds_write_b32 %0, %1\n\t"
                "ds_write_b32 %0, %2 offset:256\n\t"
                "ds_write_b32 %0, %3 offset:512"
                :
                : "v"(sbase + 4 * lane), "v"(d0), "v"(d1), "v"(d2)
                : "memory");
            if ((lane & 7) == 0)
                asm volatile("ds_write_b32 %0, %1 offset:768"
                             :
                             : "v"(sbase + 4 * (lane >> 3)), "v"(__float_as_int((float)sx * scale))
                             : "memory");
            if (lane == 0)
                asm volatile("ds_write_b32 %0, %1 offset:832" : : "v"(sbase), "v"(__float_as_int(scale)) : "memory");
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
                    A[pp][c] = i32x4{ha == 0 ? (int)dl[c].x : 0, ha == 0 ? (int)dl[c].y : 0,
                                     ha == 1 ? (int)dh[c].x : 0, ha == 1 ? (int)dh[c].y : 0};
                }
            }
            if (tq == tj) {  // output lanes of route j
#pragma unroll
                for (int c = 0; c < 4; c++) xs4[pp][c] = xsv[c];
                xs[pp] = sc;
            }
        }
    };

    // Results of item `it` from the partial sums in part[buf]: one wave per item.
    int nout = 0;  // buffered results (every wave keeps the same count)
    auto reduce = [&](const Item &it, int buf, int base) {
        if (MODE == 0) {
            if (lane < it.ntok * 16) {
                const int tk = lane >> 4, r = lane & 15;
                if (r < it.nrows) {
                    float gs = 0.0f, us = 0.0f;
                    for (int s = 0; s < G.nsb; s++) {
                        gs += part[buf][tk][s][r];
                        us += part[buf][tk][G.nsb + s][r];
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
        nout += it.ntok * it.nrows;
    };
    auto flush = [&]() {
        __syncthreads();
        for (int q = threadIdx.x; q < nout; q += kMoThreads) out[outi[q]] = outv[q];
        nout = 0;
        __syncthreads();
    };

    // Prologue: the first group's vectors, the first items' loads, then the
    // group's operands.
    Cursor c_cur = c_first;
    Item cur = item_of(c_cur);
    build(cur, false, [&]() {
#pragma unroll
        for (int j = 0; j < kMoSlots - 1; j++) issue(j, i_begin + j);
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
        if (active) {
            u32x4 hv;
            uint2 q[4];
            const uint32_t off = (uint32_t)slot * kMoSlot;
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
            i32x4 B[4];
#pragma unroll
            for (int c = 0; c < 4; c++)
                B[c] = i32x4{(int)(q[c].x & 0x0F0F0F0Fu), (int)(q[c].y & 0x0F0F0F0Fu),
                             (int)((q[c].x >> 4) & 0x0F0F0F0Fu), (int)((q[c].y >> 4) & 0x0F0F0F0Fu)};
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
#pragma unroll
            for (int pp = 0; pp < 2; pp++) {
                if (pp >= npairs) break;  // uniform
                // the pair's four products first, then their plane combines
                i32x4 D[4];
#pragma unroll
                for (int c = 0; c < 4; c++) D[c] = __builtin_amdgcn_mfma_i32_16x16x64_i8(A[pp][c], B[c], zero4, 0, 0, 0);
                int S[4];
#pragma unroll
                for (int c = 0; c < 4; c++)
                    S[c] = (int)(((uint32_t)D[c][2] << 16) + (((uint32_t)D[c][1] << 8) + (uint32_t)D[c][0]));
                float v;
                if (fin) {
                    float qs = 0.0f, mm = 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        qs = fmaf(scf[c], (float)S[c], qs);
                        mm = fmaf(mnf[c], xs4[pp][c], mm);
                    }
                    v = fmaf(d * xs[pp], qs, -(dmin * mm));
                } else {
                    // the reference's (d sc) products; zero min codes skip a
                    // non-finite dmin (minContribution, RT/GgufKQuantLayout.java:67-69)
                    float qs = 0.0f, mm = 0.0f;
#pragma unroll
                    for (int c = 0; c < 4; c++) {
                        qs = fmaf(d * scf[c], xs[pp] * (float)S[c], qs);
                        mm = fmaf(mnf[c] != 0.0f ? dmin * mnf[c] : 0.0f, xs4[pp][c], mm);
                    }
                    v = qs - mm;
                }
                // h = 1 half of row n: lane n + 16 (ds_swizzle, lanes xor 16)
                const float other = __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
                if (h == 0) part[i & 1][2 * pp + tq][wv][n] = v + other;
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

namespace {

MoeTileGeom make_geom(int mode, int E, int H, int I) {
    MoeTileGeom g{};
    const int K = mode == 0 ? H : I;
    g.nsb = K / kQK;
    g.rows_e = mode == 0 ? I : H;
    g.rt = mode == 0 ? 1 : (16 / g.nsb);
    g.tiles_e = (g.rows_e + 16 * g.rt - 1) / (16 * g.rt);
    g.row_bytes = (uint32_t)(g.nsb * kQKBlockBytes);
    // a pitch whose 16-byte units are odd modulo 16 spreads 16 rows over all banks
    g.pitch = ((g.row_bytes / 16) % 2 == 1) ? g.row_bytes : g.row_bytes + 16;
    const int part_bytes = 16 * g.rt * (int)g.pitch;
    g.part_dma = (part_bytes + 1023) / 1024;
    g.ndma = mode == 0 ? 2 * g.part_dma : g.part_dma;
    g.vec_len = K;
    g.out_len = g.rows_e;
    g.w_bytes = (int64_t)E * g.rows_e * g.row_bytes;
    return g;
}

}  // namespace

bool moe_q4k_mfma_supported(int E, int H, int I, const float *x) {
    if (H % kQK != 0 || I % kQK != 0 || H > 8 * kQK || I > 16 * kQK) return false;
    if ((reinterpret_cast<uintptr_t>(x) & 15u) != 0) return false;
    for (int mode = 0; mode < 2; mode++) {
        const MoeTileGeom g = make_geom(mode, E, H, I);
        if (g.ndma > kMoMaxDma || g.w_bytes >= (int64_t)kMaskedOffset) return false;
        if (2 * kMoGroup * 16 * g.rt > kMoOutCap) return false;
    }
    return true;
}

// Routing, gate/up, down and combine (4 launches); the caller has checked
// moe_q4k_mfma_supported.
hipError_t launch_moe_q4k_mfma(const uint8_t *gate, const uint8_t *up, const uint8_t *down, int E,
                               int H, int I, const float *x, const int32_t *ids, const float *wts,
                               int T, int top_k, float *out, uint8_t *ws, hipStream_t stream) {
    const MoeLayout L = moe_layout(T, top_k, H, I, E);
    const int P = T * top_k;
    int32_t *meta = reinterpret_cast<int32_t *>(ws + L.meta);
    const MoeTileGeom g0 = make_geom(0, E, H, I), g1 = make_geom(1, E, H, I);
    hipError_t e = launch_moe_route(ids, wts, P, E, g0.tiles_e, g1.tiles_e, meta, stream);
    if (e != hipSuccess) return e;
    const unsigned grid = (unsigned)device_cus();
    float *hbuf = reinterpret_cast<float *>(ws + L.h);
    float *ypair = reinterpret_cast<float *>(ws + L.ypair);
    hipLaunchKernelGGL(moe_expert_tile_kernel<0>, dim3(grid), dim3(kMoThreads), 0, stream, gate, up, g0, x,
                       top_k, meta, E, P, hbuf);
    hipLaunchKernelGGL(moe_expert_tile_kernel<1>, dim3(grid), dim3(kMoThreads), 0, stream, down,
                       (const uint8_t *)nullptr, g1, (const float *)hbuf, top_k, meta, E, P, ypair);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
    return launch_moe_combine(ids, wts, ypair, T, top_k, H, E, out, stream);
}

}  // namespace gollek
