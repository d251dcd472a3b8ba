// gguf_moe.hip -- grouped MoE expert FFN on gfx950: the dispatch by expert
// type and shape, the routing and route-order combine kernels, and the
// passes that do not use the matrix cores (gguf_moe_mfma.hip has those).
//
// Semantics of runner/safetensor/gollek-safetensor-engine/src/main/java/tech/
// kayys/gollek/safetensor/engine/generation/moe/MoeForwardPass.java:217-240 and
// :461-472 (MFP below): for each token t and each of its top-k routes j,
//   out[t] += w[t,j] * down_e(silu(gate_e x_t) * up_e x_t),   e = ids[t,j],
// accumulated in routing order; routes with an out-of-range expert id or a
// zero weight are skipped (MFP:222).  swigluFfn = down(silu(gate x) * up x)
// (.../engine/forward/DirectForwardFfnService.java:40-61).  Expert weights are
// GGUF Q4_0 / Q8_0 / Q4_K / Q5_K / Q6_K, stacked the way GGUF stores experts:
// gate/up have experts * inter rows of `hidden` columns, down has experts *
// hidden rows of `inter` columns.
//
// The reference runs every (token, route) pair separately and so re-reads an
// expert's weights once per pair.  Here the pairs are grouped by expert on the
// device and every used expert's weights stream from HBM once per group of
// up to four of its routes:
//   1. route: count pairs per expert, stable-sort the pair list by expert,
//      list the used experts (one workgroup);
//   2. gate/up: per (used expert, row tile) the gate and up rows are loaded
//      once and contracted against the expert's routes; h = silu(g) u;
//   3. down: per (used expert, row tile), y_pair = down_e h;
//   4. combine: out[t] = sum_j w[t,j] y_pair[t,j] in j order (plain fp32
//      multiply then add, as MFP:461-472 accumulates).
// Passes 2 and 3 per type: Q8_0 / Q4_0 rows on moe_q32_expert_kernel, Q4_K /
// Q5_K / Q6_K rows on moe_kq_expert_kernel (fp32, the routes' vectors staged
// in LDS), all-Q4_K layers up to hidden 4096 on the v_dot4 kernels
// (moe_expert_kernel, x and h as integer digit planes, gguf_dot4.hpp), and
// anything else on moe_generic_expert_kernel (byte loads, any alignment).
// launch_moe sends the shapes the matrix-core passes take there first
// (more than 2048 routes as token slices of at most 2048 / top_k tokens).
#include "gguf_block_dot.hpp"
#include "gguf_dot4.hpp"
#include "gguf_kernels.hpp"

namespace gollek {

namespace {

constexpr int kMoeTokensPerPass = 8;  // vectors staged in LDS at once

size_t align256(size_t v) { return (v + 255) / 256 * 256; }

}  // namespace

// meta (int32): counts[E] | offsets[E+1] | pairs[P] | used[E] | nused |
// items0[E+1] | items1[E+1] (work-item offsets of the used experts for the
// gate/up and down passes of the matrix-core kernels)
MoeLayout moe_layout(int64_t tokens, int64_t top_k, int64_t hidden, int64_t inter,
                     int64_t experts) {
    MoeLayout L;
    const int64_t P = tokens * top_k;
    L.meta_ints = 2 * experts + 1 + P + experts + 1 + 2 * (experts + 1);
    L.meta = 0;
    L.xdig = align256(L.meta + (size_t)L.meta_ints * 4);
    L.xdig_stride = align256(digit_lds_bytes((int)(hidden / 32)));
    L.h = align256(L.xdig + (size_t)tokens * L.xdig_stride);
    L.hdig = align256(L.h + (size_t)P * inter * 4);
    L.hdig_stride = align256(digit_lds_bytes((int)(inter / 32)));
    L.ypair = align256(L.hdig + (size_t)P * L.hdig_stride);
    L.total = align256(L.ypair + (size_t)P * hidden * 4);
    return L;
}

// Routing on one workgroup: per-expert counts of the valid routes (expert id
// in range, weight != 0; MFP:222), their offsets, the route list stably
// sorted by expert, the used experts in expert order, and per used expert
// u the work-item offsets items0/items1 = prefix of tiles * ceil(count / 4)
// for the two expert passes.  Wave 0 scans in chunks of 64 with DPP-free
// shuffles; the stable scatter ranks equal keys within a chunk by ballots.
__global__ __launch_bounds__(256) void moe_route_kernel(const int32_t *__restrict__ ids,
                                                        const float *__restrict__ wts, int P,
                                                        int E, int tiles0, int tiles1,
                                                        int32_t *__restrict__ meta, int keys_in_lds) {
    extern __shared__ int32_t sh[];  // cnt[E], run[E], then (keys_in_lds) key[P]
    int32_t *cnt = sh, *run = sh + E, *keys = sh + 2 * E;
    int32_t *counts = meta, *offsets = meta + E, *pairs = meta + 2 * E + 1;
    int32_t *used = pairs + P, *nused = used + E;
    int32_t *items0 = nused + 1, *items1 = items0 + E + 1;
    const int lane = threadIdx.x & 63;
    for (int e = threadIdx.x; e < E; e += blockDim.x) cnt[e] = 0;
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += blockDim.x) {
        const int e = ids[p];
        const bool valid = e >= 0 && e < E && wts[p] != 0.0f;
        if (valid) atomicAdd(&cnt[e], 1);  // LDS atomic
        if (keys_in_lds) keys[p] = valid ? e : -1;
    }
    __syncthreads();
    if (threadIdx.x < 64) {
        const uint64_t below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
        int carry = 0, ucount = 0, it0 = 0, it1 = 0;
        for (int base = 0; base < E; base += 64) {
            const int e = base + lane;
            const int c = e < E ? cnt[e] : 0;
            const int groups = (c + 3) / 4;
            int a = c, b0 = tiles0 * groups, b1 = tiles1 * groups;
            // inclusive scans over the 64 lanes
            for (int d = 1; d < 64; d <<= 1) {
                const int ta = __shfl_up(a, d, 64), tb0 = __shfl_up(b0, d, 64), tb1 = __shfl_up(b1, d, 64);
                if (lane >= d) {
                    a += ta;
                    b0 += tb0;
                    b1 += tb1;
                }
            }
            const uint64_t ub = __ballot(c > 0);
            if (e < E) {
                offsets[e] = carry + a - c;
                counts[e] = c;
                run[e] = carry + a - c;
            }
            if (c > 0) {
                const int u = ucount + __popcll(ub & below);
                used[u] = e;
                items0[u] = it0 + b0 - tiles0 * groups;
                items1[u] = it1 + b1 - tiles1 * groups;
            }
            carry += __shfl(a, 63, 64);
            it0 += __shfl(b0, 63, 64);
            it1 += __shfl(b1, 63, 64);
            ucount += __popcll(ub);
        }
        if (lane == 0) {
            offsets[E] = carry;
            *nused = ucount;
            items0[ucount] = it0;
            items1[ucount] = it1;
        }
        // Stable scatter, 64 routes at a time in route order: a route's slot is
        // its expert's running offset plus its rank among the chunk's equal keys.
        int bits = 1;
        while ((1 << bits) <= E) bits++;
        for (int base = 0; base < P; base += 64) {
            const int p = base + lane;
            int key = -1;
            if (p < P) {
                if (keys_in_lds) {
                    key = keys[p];
                } else {
                    const int e = ids[p];
                    if (e >= 0 && e < E && wts[p] != 0.0f) key = e;
                }
            }
            const uint32_t k1 = (uint32_t)(key + 1);
            uint64_t same = __ballot(true);
            for (int bt = 0; bt < bits; bt++) {
                const uint64_t v = __ballot((k1 >> bt) & 1u);
                same &= ((k1 >> bt) & 1u) ? v : ~v;
            }
            const int rank = __popcll(same & below);
            const int r0 = key >= 0 ? run[key] : 0;  // read by all lanes before any update
            if (key >= 0) pairs[r0 + rank] = p;
            const bool last = (same >> lane) == 1ull;  // highest lane of its key
            if (key >= 0 && last) run[key] = r0 + __popcll(same);
        }
    }
}

// Digit planes of `count` vectors of `len` floats, one workgroup per vector.
__global__ __launch_bounds__(256) void moe_digits_kernel(const float *__restrict__ v, int len,
                                                         int64_t v_stride, uint8_t *__restrict__ dig,
                                                         int64_t dig_stride) {
    const int ngroups = len / 32;
    uint32_t *d = reinterpret_cast<uint32_t *>(dig + (int64_t)blockIdx.x * dig_stride);
    float *scl = reinterpret_cast<float *>(d + kDigitWords * ngroups);
    build_x_digits(v + (int64_t)blockIdx.x * v_stride, ngroups, d, scl, scl + ngroups);
}

// Rows [r0, r_end) of expert e (of one or two stacked matrices) against the
// expert's vectors.  GATED: out[p][r] = silu(w0 . v) * (w1 . v), else
// out[p][r] = w0 . v.  Vector of pair p: digits[by_pair ? p : p / top_k].
template <int LPR, bool GATED, int RB>
__global__ __launch_bounds__(256) void moe_expert_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, int64_t row_bytes, int nsb,
    int rows_per_expert, int rows_per_block, const uint8_t *__restrict__ digits,
    int64_t digit_stride, int by_pair, int top_k, const int32_t *__restrict__ meta, int E, int P,
    float *__restrict__ out, int64_t out_stride) {
    extern __shared__ uint32_t smem[];
    constexpr int RG = 64 / LPR;
    const int32_t *counts = meta, *offsets = meta + E, *pairs = meta + 2 * E + 1;
    const int32_t *used = pairs + P;
    const int nused = used[E];
    if ((int)blockIdx.y >= nused) return;  // uniform: before any barrier
    const int e = used[blockIdx.y];
    const int cnt = counts[e], p0 = offsets[e];
    const int ngroups = nsb * 8;
    const int vec_words = (int)(digit_stride / 4);

    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int rg = lane / LPR, gl = lane & (LPR - 1), g = gl & 3, sb = gl >> 2;
    const bool act = sb < nsb;
    const int r_lo = blockIdx.x * rows_per_block;
    const int r_hi = min(rows_per_expert, r_lo + rows_per_block);
    const int rows_per_wave = (rows_per_block + 3) / 4;
    const int wr0 = r_lo + wave * rows_per_wave;
    const int wr1 = min(r_hi, wr0 + rows_per_wave);
    const uint8_t *w0e = w0 + (int64_t)e * rows_per_expert * row_bytes;
    const uint8_t *w1e = GATED ? w1 + (int64_t)e * rows_per_expert * row_bytes : nullptr;

    for (int c0 = 0; c0 < cnt; c0 += kMoeTokensPerPass) {
        const int tc = min(kMoeTokensPerPass, cnt - c0);
        __syncthreads();
        // Stage the digit planes of vectors c0 .. c0 + tc into LDS.
        for (int j = 0; j < tc; j++) {
            const int p = pairs[p0 + c0 + j];
            const int vi = by_pair ? p : p / top_k;
            const uint4 *src = reinterpret_cast<const uint4 *>(digits + (int64_t)vi * digit_stride);
            uint4 *dst = reinterpret_cast<uint4 *>(smem + j * vec_words);
            for (int i = threadIdx.x; i < vec_words / 4; i += blockDim.x) dst[i] = src[i];
        }
        __syncthreads();
        for (int r0 = wr0; r0 < wr1; r0 += RG * RB) {
            RowChunk A[RB], B[RB];
            load_rows<RB, RG>(A, w0e, row_bytes, r0, wr1, rg, sb, g, act);
            if (GATED) load_rows<RB, RG>(B, w1e, row_bytes, r0, wr1, rg, sb, g, act);
            for (int j = 0; j < tc; j++) {
                const uint32_t *dig = smem + j * vec_words;
                const float *scl = reinterpret_cast<const float *>(dig + kDigitWords * ngroups);
                uint32_t dg[2][3][8];
                float sg[2], xg[2];
                load_lane_digits(dig, scl, scl + ngroups, sb, g, act, dg, sg, xg);
                const int p = pairs[p0 + c0 + j];
                float res[RB];
#pragma unroll
                for (int i = 0; i < RB; i++) {
                    float a = group_sum<LPR>(q4k_dot4_row(A[i].h, A[i].a, A[i].b, dg, sg, xg, g));
                    if (GATED) {
                        const float b = group_sum<LPR>(q4k_dot4_row(B[i].h, B[i].a, B[i].b, dg, sg, xg, g));
                        a = a / (1.0f + expf(-a)) * b;  // silu(gate) * up
                    }
                    res[i] = a;
                }
                if (gl == 0) {
#pragma unroll
                    for (int i = 0; i < RB; i++) {
                        const int r = r0 + i * RG + rg;
                        if (r < wr1) out[(int64_t)p * out_stride + r] = res[i];
                    }
                }
            }
        }
    }
}

// out[t][c] = sum_j w[t,j] * y[t*k + j][c] over valid routes, j in order.
// Eight routes at a time: their ids and weights, then their rows (every
// route's row is in the workspace, so an invalid route's load is in bounds
// and its value is dropped by a select), then the sums in route order --
// one memory round trip per eight routes instead of two per route.
__global__ __launch_bounds__(256) void moe_combine_kernel(const int32_t *__restrict__ ids,
                                                          const float *__restrict__ wts,
                                                          const float *__restrict__ ypair, int T,
                                                          int top_k, int H, int E,
                                                          float *__restrict__ out) {
#pragma clang fp contract(off)
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)T * H) return;
    const int t = (int)(i / H), c = (int)(i % H);
    float acc = 0.0f;
    for (int j0 = 0; j0 < top_k; j0 += 8) {
        bool ok[8];
        float wj[8], yv[8];
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u < top_k ? j0 + u : top_k - 1;
            const int p = t * top_k + j;
            const int e = ids[p];
            wj[u] = wts[p];
            ok[u] = j0 + u < top_k && e >= 0 && e < E && wj[u] != 0.0f;
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const int j = j0 + u < top_k ? j0 + u : top_k - 1;
            yv[u] = ypair[(int64_t)(t * top_k + j) * H + c];
        }
#pragma unroll
        for (int u = 0; u < 8; u++) {
            const float scaled = yv[u] * wj[u];  // AccelOps.mulScalar
            acc = ok[u] ? acc + scaled : acc;    // addToTokenRow
        }
    }
    out[i] = acc;
}

// The shared expert's routes: every token to expert 0 with weight 1.
__global__ __launch_bounds__(256) void moe_shared_routes_kernel(int32_t *__restrict__ ids,
                                                                float *__restrict__ wts, int T) {
    const int t = (int)(blockIdx.x * blockDim.x + threadIdx.x);
    if (t < T) {
        ids[t] = 0;
        wts[t] = 1.0f;
    }
}

// The shared expert added after token t's routes (MoeForwardPass.java:240-247):
// out[t] = out[t] + g * y[t], the product rounded first (AccelOps.mulScalar,
// then addToTokenRow).  g = 1 / (1 + (float)exp(-s)) in float with exp in
// double (resolveSharedExpertGate, :428-442), s = x_t . gate_inp rounded
// to float (the sum in fp64, whose products of two floats are exact); g = 1
// without gate_inp.  One workgroup per token.
__global__ __launch_bounds__(256) void moe_shared_add_kernel(const float *__restrict__ x,
                                                             const float *__restrict__ gate_inp,
                                                             const float *__restrict__ y, int H,
                                                             float *__restrict__ out) {
#pragma clang fp contract(off)
    __shared__ double part[4];
    const int t = (int)blockIdx.x;
    const int64_t row = (int64_t)t * H;
    float g = 1.0f;
    if (gate_inp != nullptr) {  // uniform
        double s = 0.0;
        for (int i = (int)threadIdx.x; i < H; i += 256) s += (double)x[row + i] * (double)gate_inp[i];
        for (int off = 32; off > 0; off >>= 1) s += __shfl_xor(s, off);
        if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = s;
        __syncthreads();
        const float sf = (float)(((part[0] + part[1]) + part[2]) + part[3]);
        g = 1.0f / (1.0f + (float)exp((double)(-sf)));
    }
    for (int i = (int)threadIdx.x; i < H; i += 256) {
        const float scaled = g * y[row + i];
        out[row + i] = out[row + i] + scaled;
    }
}

// Any expert types (Q8_0, Q4_0, Q4_K, Q5_K, Q6_K), any alignment: rows
// [r0, r0 + rows_per_block) of expert e against each of the expert's
// vectors, one wave per row and one lane per block (fp32, byte loads).
// GATED: out[p][r] = silu(w0 . v) * (w1 . v) with w0, w1 of types t0, t1,
// else out[p][r] = w0 . v.  Vector of pair p: vec[(by_pair ? p : p / top_k)
// * vec_stride].  The expert's rows are re-read per route from the caches.
template <bool GATED>
__global__ __launch_bounds__(256) void moe_generic_expert_kernel(
    int t0, int t1, const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, int64_t rb0,
    int64_t rb1, int cols, int rows_per_expert, int rows_per_block, const float *__restrict__ vec,
    int64_t vec_stride, int by_pair, int top_k, const int32_t *__restrict__ meta, int E, int P,
    float *__restrict__ out, int64_t out_stride) {
    const int32_t *counts = meta, *offsets = meta + E, *pairs = meta + 2 * E + 1;
    const int32_t *used = pairs + P;
    if ((int)blockIdx.y >= used[E]) return;
    const int e = used[blockIdx.y];
    const int cnt = counts[e], p0 = offsets[e];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int bs0 = block_elems(t0), bb0 = block_bytes(t0), bs1 = block_elems(t1), bb1 = block_bytes(t1);
    const int nb0 = cols / bs0, nb1 = GATED ? cols / bs1 : 0;
    const int r_lo = blockIdx.x * rows_per_block;
    const int r_hi = min(rows_per_expert, r_lo + rows_per_block);
    for (int r = r_lo + wave; r < r_hi; r += 4) {
        const uint8_t *row0 = w0 + ((int64_t)e * rows_per_expert + r) * rb0;
        const uint8_t *row1 = GATED ? w1 + ((int64_t)e * rows_per_expert + r) * rb1 : nullptr;
        for (int c = 0; c < cnt; c++) {
            const int p = pairs[p0 + c];
            const float *v = vec + (int64_t)(by_pair ? p : p / top_k) * vec_stride;
            float a = 0.0f;
            for (int b = lane; b < nb0; b += 64) a += generic_block_dot(t0, row0 + (int64_t)b * bb0, v + b * bs0);
            a = group_sum<64>(a);
            if (GATED) {
                float u = 0.0f;
                for (int b = lane; b < nb1; b += 64) u += generic_block_dot(t1, row1 + (int64_t)b * bb1, v + b * bs1);
                u = group_sum<64>(u);
                a = a / (1.0f + expf(-a)) * u;  // silu(gate) * up
            }
            if (lane == 0) out[(int64_t)p * out_stride + r] = a;
        }
    }
}

// Q8_0 / Q4_0 expert rows against the vectors of up to four routes of the
// expert at a time.  The routes' vectors are staged in LDS, 36 floats per
// 32-element block: the block's 32 values, then (Q4_0) their sum, which
// takes the codes' offset of 8 out as -8 sum(x); the padding also puts the
// blocks that neighbouring lanes read on distinct banks.  LPR lanes per row
// (64 / LPR rows of a wave at a time), lane s of a row taking blocks s,
// s + LPR, ... in chunks of KPL blocks whose bytes are loaded together (dword
// loads through a buffer descriptor over the expert's rows, realigned by the
// block's offset within a dword).  Each block's codes are widened once and
// contracted with every staged route in fp32: d * sum(q x) per block, as the
// reference's block dot.  GATED: the expert's gate and up rows r,
// h = silu(gate . x) * (up . x).
template <int T>
struct Q32Raw {
    static constexpr int kDw = T == kQ8_0 ? 9 : 5;  // dwords covering a block from its offset & ~3
    uint32_t w[kDw];
};

// Default cache policy, as for the K-quant rows below: a block's dword loads
// revisit its lines (streaming hints: 162 against 119 us for a Q8_0 layer).
template <int T>
__device__ __forceinline__ void q32_load(__amdgpu_buffer_rsrc_t rs, uint32_t off, Q32Raw<T> &r) {
    const uint32_t base = off & ~3u;
#pragma unroll
    for (int i = 0; i < Q32Raw<T>::kDw; i++)
        r.w[i] = __builtin_amdgcn_raw_buffer_load_b32(rs, base + 4u * i, 0, 0);
}

// The block's codes as floats (Q4_0: the nibble 0..15, without the -8) and d;
// sh = the block's byte offset within its first dword (0 or 2: blocks start
// at even bytes).
template <int T>
__device__ __forceinline__ void q32_codes(const Q32Raw<T> &r, uint32_t sh, float (&q)[32], float &d) {
    d = half_bits_to_float_fast(sh ? r.w[0] >> 16 : r.w[0] & 0xFFFFu);
    constexpr int kQd = T == kQ8_0 ? 8 : 4;  // code dwords
    uint32_t c[kQd];
#pragma unroll
    for (int i = 0; i < kQd; i++) c[i] = sh ? r.w[i + 1] : __builtin_amdgcn_alignbyte(r.w[i + 1], r.w[i], 2);
    if constexpr (T == kQ8_0) {
#pragma unroll
        for (int i = 0; i < 8; i++)
#pragma unroll
            for (int k = 0; k < 4; k++) q[4 * i + k] = sbyte_f(c[i], k);
    } else {
        // element j < 16: low nibble of code byte j; j >= 16: high nibble of byte j - 16
#pragma unroll
        for (int i = 0; i < 4; i++)
#pragma unroll
            for (int k = 0; k < 4; k++) {
                q[4 * i + k] = byte_f(c[i] & 0x0F0F0F0Fu, k);
                q[16 + 4 * i + k] = byte_f((c[i] >> 4) & 0x0F0F0F0Fu, k);
            }
    }
}

constexpr int kQ32Group = 4;

template <int T, bool GATED, int LPR>
__global__ __launch_bounds__(256) void moe_q32_expert_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, int64_t row_bytes, int cols,
    int rows_per_expert, int rows_per_block, const float *__restrict__ vec, int64_t vec_stride, int by_pair,
    int top_k, const int32_t *__restrict__ meta, int E, int P, int group, float *__restrict__ out,
    int64_t out_stride) {
    extern __shared__ float xs[];  // group x nb x 36 floats
    constexpr int kBB = T == kQ8_0 ? 34 : 18;
    constexpr int KPL = (T == kQ8_0 && GATED) ? 2 : 4;  // blocks a lane loads together
    constexpr int RPW = 64 / LPR;                         // rows of a wave at a time
    const int32_t *counts = meta, *offsets = meta + E, *pairs = meta + 2 * E + 1;
    const int32_t *used = pairs + P;
    if ((int)blockIdx.y >= used[E]) return;
    const int e = used[blockIdx.y];
    const int cnt = counts[e], p0 = offsets[e];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int nb = cols / 32, c4 = cols / 4;
    const int r_lo = blockIdx.x * rows_per_block;
    const int r_hi = min(rows_per_expert, r_lo + rows_per_block);
    const int64_t ebytes = (int64_t)rows_per_expert * row_bytes;
    const __amdgpu_buffer_rsrc_t rs0 = wave_buffer(w0 + (int64_t)e * ebytes, (uint32_t)ebytes);
    const __amdgpu_buffer_rsrc_t rs1 = wave_buffer((GATED ? w1 : w0) + (int64_t)e * ebytes, (uint32_t)ebytes);
    for (int g0 = 0; g0 < cnt; g0 += group) {
        const int gn = min(group, cnt - g0);
        __syncthreads();  // the previous group's vectors are no longer read
        for (int i = threadIdx.x; i < gn * c4; i += 256) {
            const int q = i / c4, j = 4 * (i - q * c4);
            const int p = pairs[p0 + g0 + q];
            const float4 v = *reinterpret_cast<const float4 *>(vec + (int64_t)(by_pair ? p : p / top_k) * vec_stride + j);
            *reinterpret_cast<float4 *>(xs + (q * nb + (j >> 5)) * 36 + (j & 31)) = v;
        }
        if constexpr (T == kQ4_0) {
            __syncthreads();
            for (int i = threadIdx.x; i < gn * nb; i += 256) {
                const float *xb = xs + i * 36;
                float t = 0.0f;
                for (int k = 0; k < 32; k++) t += xb[k];
                xs[i * 36 + 32] = t;
            }
        }
        __syncthreads();
        for (int r0 = r_lo + wave * RPW; r0 < r_hi; r0 += 4 * RPW) {
            const int r = r0 + rsub;
            const bool live = r < r_hi;
            const uint32_t row_off = live ? (uint32_t)((int64_t)r * row_bytes) : 0u;
            float a[kQ32Group], u[kQ32Group];
#pragma unroll
            for (int q = 0; q < kQ32Group; q++) a[q] = u[q] = 0.0f;
            for (int b0 = 0; b0 < nb; b0 += KPL * LPR) {
                Q32Raw<T> raw0[KPL], raw1[KPL];
#pragma unroll
                for (int k = 0; k < KPL; k++) {
                    const int b = b0 + sub + LPR * k;
                    if (live && b < nb) {
                        q32_load<T>(rs0, row_off + (uint32_t)(b * kBB), raw0[k]);
                        if constexpr (GATED) q32_load<T>(rs1, row_off + (uint32_t)(b * kBB), raw1[k]);
                    }
                }
#pragma unroll
                for (int k = 0; k < KPL; k++) {
                    const int b = b0 + sub + LPR * k;
                    if (!(live && b < nb)) continue;
                    const uint32_t sh = (row_off + (uint32_t)(b * kBB)) & 3u;
                    float cq[32], d0, cu[32], d1 = 0.0f;
                    q32_codes<T>(raw0[k], sh, cq, d0);
                    if constexpr (GATED) q32_codes<T>(raw1[k], sh, cu, d1);
#pragma unroll
                    for (int q = 0; q < kQ32Group; q++) {
                        if (q < gn) {
                            const float4 *xb = reinterpret_cast<const float4 *>(xs + (q * nb + b) * 36);
                            float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                            for (int i = 0; i < 8; i++) {
                                const float4 xv = xb[i];
                                s0 = fmaf(cq[4 * i], xv.x, s0);
                                s0 = fmaf(cq[4 * i + 1], xv.y, s0);
                                s0 = fmaf(cq[4 * i + 2], xv.z, s0);
                                s0 = fmaf(cq[4 * i + 3], xv.w, s0);
                                if constexpr (GATED) {
                                    s1 = fmaf(cu[4 * i], xv.x, s1);
                                    s1 = fmaf(cu[4 * i + 1], xv.y, s1);
                                    s1 = fmaf(cu[4 * i + 2], xv.z, s1);
                                    s1 = fmaf(cu[4 * i + 3], xv.w, s1);
                                }
                            }
                            if constexpr (T == kQ4_0) {
                                const float xsum = xs[(q * nb + b) * 36 + 32];
                                s0 = fmaf(-8.0f, xsum, s0);
                                if constexpr (GATED) s1 = fmaf(-8.0f, xsum, s1);
                            }
                            a[q] = fmaf(d0, s0, a[q]);
                            if constexpr (GATED) u[q] = fmaf(d1, s1, u[q]);
                        }
                    }
                }
            }
#pragma unroll
            for (int q = 0; q < kQ32Group; q++) {
                if (q < gn) {
                    float v = group_sum<LPR>(a[q]);
                    if constexpr (GATED) {
                        const float uu = group_sum<LPR>(u[q]);
                        v = v / (1.0f + expf(-v)) * uu;  // silu(gate) * up
                    }
                    if (sub == 0 && live) out[(int64_t)pairs[p0 + g0 + q] * out_stride + r] = v;
                }
            }
        }
    }
}

// K-quant (Q4_K, Q5_K, Q6_K) expert rows, in the form of the Q8_0 / Q4_0
// row kernel above: up to four routes' vectors staged in LDS at 36 floats
// per 32 elements, each group's two 16-element sums in its padding (the
// min terms and Q6_K's -32 take sums of x); LPR lanes per row, lane s taking
// superblocks s, s + LPR, ...; routes one at a time; a superblock's bytes
// (gate's and up's together) are loaded as dwords through a buffer
// descriptor (Q6_K's 210-byte superblocks realigned when they start 2 bytes
// into a dword) and its codes widened as they are contracted in fp32, with the per-sub-block scales and mins of the
// reference's dequantizers (RT/GgufKBlockDequantizer.java:31-170, 319-432)
// folded into the dot as in gguf_block_dot.hpp.
// Default cache policy: each 128-byte line is read by several of a lane's
// loads in turn (a superblock spans lines, a line several superblocks'
// pieces), and a streaming hint had each load fetch its line again (227
// against 76 us for the loads of a Q5_K / Q6_K layer).
__device__ __forceinline__ uint32_t kq_ld(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_amdgcn_raw_buffer_load_b32(rs, off, 0, 0);
}

// sum over 4 codes (bytes of q4, values 0..63) times 4 staged x values
__device__ __forceinline__ float kq_dot4(uint32_t q4, float4 xv, float s) {
    s = fmaf(byte_f(q4, 0), xv.x, s);
    s = fmaf(byte_f(q4, 1), xv.y, s);
    s = fmaf(byte_f(q4, 2), xv.z, s);
    return fmaf(byte_f(q4, 3), xv.w, s);
}

// A superblock's dwords from its offset & ~3 (Q6_K's 210-byte superblocks
// start 0 or 2 bytes into a dword; the others are 16-byte aligned).
template <int T>
struct KqRaw {
    static constexpr int kDw = T == kQ4_K ? 36 : T == kQ5_K ? 44 : 54;
    uint32_t w[kDw];
};

template <int T>
__device__ __forceinline__ void kq_load(__amdgpu_buffer_rsrc_t rs, uint32_t off, KqRaw<T> &r) {
    const uint32_t base = off & ~3u;
#pragma unroll
    for (int i = 0; i < KqRaw<T>::kDw; i++) r.w[i] = kq_ld(rs, base + 4u * i);
}

// One superblock (its dwords in r, realigned in place for Q6_K; sh = its
// offset within the first dword) against one route's staged x (xg: its 8
// groups of 36 floats).  The 64- (32-) element chunks run in a loop that is
// not unrolled, each picking its code dwords from the registers with one
// select, so only one chunk's x is held at a time.
template <int T>
__device__ __forceinline__ float kq_dot(KqRaw<T> &r, uint32_t sh, const float *xg) {
    if constexpr (T == kQ6_K) {
#pragma unroll
        for (int k = 0; k < 53; k++) r.w[k] = __builtin_amdgcn_alignbyte(r.w[k + 1], r.w[k], sh);
        const float d = half_bits_to_float_fast(r.w[52] & 0xFFFFu);
        float total = 0.0f;
#pragma unroll
        for (int h = 0; h < 2; h++) {
#pragma unroll 1
            for (int j = 0; j < 4; j++) {
                // elements 128 h + 32 j + i: ql byte 64 h + 32 (j & 1) + i, nibble j >> 1;
                // qh byte 128 + 32 h + i, bits 2 j
                const int grp = 4 * h + j;
                const float4 *xb = reinterpret_cast<const float4 *>(xg + 36 * grp);
                const uint32_t nsh = 4u * (uint32_t)(j >> 1), hsh = 2u * (uint32_t)j;
                float s0 = 0.0f, s1 = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t ql = (j & 1) ? r.w[16 * h + 8 + k] : r.w[16 * h + k];
                    const uint32_t qh = r.w[32 + 8 * h + k];
                    const uint32_t q4 = ((ql >> nsh) & 0x0F0F0F0Fu) | (((qh >> hsh) & 0x03030303u) << 4);
                    if (k < 4) s0 = kq_dot4(q4, xb[k], s0);
                    else s1 = kq_dot4(q4, xb[k], s1);
                }
                // scale bytes 2 grp, 2 grp + 1 (dword 48 + 2 h + (j >> 1))
                const uint32_t scd = (j >> 1) ? r.w[48 + 2 * h + 1] : r.w[48 + 2 * h];
                const float sc0 = sbyte_f(scd, 2 * (j & 1)), sc1 = sbyte_f(scd, 2 * (j & 1) + 1);
                s0 = fmaf(-32.0f, xg[36 * grp + 32], s0);
                s1 = fmaf(-32.0f, xg[36 * grp + 33], s1);
                total = fmaf(d * sc0, s0, total);
                total = fmaf(d * sc1, s1, total);
            }
        }
        return total;
    } else {
        (void)sh;
        constexpr bool q5 = T == kQ5_K;
        constexpr int qs = q5 ? 12 : 4;  // first quant dword
        const float d = half_bits_to_float_fast(r.w[0] & 0xFFFFu);
        const float dmin = half_bits_to_float_fast(r.w[0] >> 16);
        float total = 0.0f;
#pragma unroll
        for (int c2 = 0; c2 < 2; c2++) {
#pragma unroll 1
            for (int c1 = 0; c1 < 2; c1++) {
                const int c = 2 * c2 + c1;  // sub-blocks 2c, 2c + 1
                uint32_t scp, mnp;
                q4k_pair_codes(r.w[1], r.w[2], r.w[3], c, &scp, &mnp);
                const float4 *x1 = reinterpret_cast<const float4 *>(xg + 36 * (2 * c));
                const float4 *x2 = reinterpret_cast<const float4 *>(xg + 36 * (2 * c + 1));
                float a1 = 0.0f, a2 = 0.0f;
#pragma unroll
                for (int k = 0; k < 8; k++) {
                    const uint32_t qd = c1 ? r.w[qs + 8 * (2 * c2 + 1) + k] : r.w[qs + 8 * (2 * c2) + k];
                    uint32_t lo = qd & 0x0F0F0F0Fu, hi = (qd >> 4) & 0x0F0F0F0Fu;
                    if constexpr (q5) {
                        const uint32_t qh = r.w[4 + k];  // qh bytes 4 k .. 4 k + 3
                        lo |= ((qh >> (2 * c)) & 0x01010101u) << 4;
                        hi |= ((qh >> (2 * c + 1)) & 0x01010101u) << 4;
                    }
                    a1 = kq_dot4(lo, x1[k], a1);
                    a2 = kq_dot4(hi, x2[k], a2);
                }
                const float sc1 = (float)(scp & 0xFFu), sc2 = (float)((scp >> 8) & 0xFFu);
                const uint32_t mc1 = mnp & 0xFFu, mc2 = (mnp >> 8) & 0xFFu;
                const float m1 = mc1 ? dmin * (float)mc1 : 0.0f, m2 = mc2 ? dmin * (float)mc2 : 0.0f;
                const float v1 = xg[36 * (2 * c) + 32] + xg[36 * (2 * c) + 33];
                const float v2 = xg[36 * (2 * c + 1) + 32] + xg[36 * (2 * c + 1) + 33];
                total += d * sc1 * a1 + d * sc2 * a2 - (m1 * v1 + m2 * v2);
            }
        }
        return total;
    }
}

template <int T, bool GATED, int LPR>
__global__ __launch_bounds__(256) void moe_kq_expert_kernel(
    const uint8_t *__restrict__ w0, const uint8_t *__restrict__ w1, int64_t row_bytes, int cols,
    int rows_per_expert, int rows_per_block, const float *__restrict__ vec, int64_t vec_stride, int by_pair,
    int top_k, const int32_t *__restrict__ meta, int E, int P, int group, float *__restrict__ out,
    int64_t out_stride) {
    // group x (cols / 32 groups of 36 floats, plus 4 after every 8 groups:
    // superblocks 292 floats apart, so the lanes of a row, one superblock
    // each, read distinct banks)
    extern __shared__ float xs[];
    constexpr int kSB = T == kQ4_K ? 144 : T == kQ5_K ? 176 : 210;
    constexpr int RPW = 64 / LPR;  // rows of a wave at a time
    const int32_t *counts = meta, *offsets = meta + E, *pairs = meta + 2 * E + 1;
    const int32_t *used = pairs + P;
    if ((int)blockIdx.y >= used[E]) return;
    const int e = used[blockIdx.y];
    const int cnt = counts[e], p0 = offsets[e];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int sub = lane % LPR, rsub = lane / LPR;
    const int ng = cols / 32, nsb = cols / 256, c4 = cols / 4;
    const int rstride = ng * 36 + nsb * 4;  // floats per route
    auto goff = [&](int g) { return g * 36 + (g >> 3) * 4; };
    const int r_lo = blockIdx.x * rows_per_block;
    const int r_hi = min(rows_per_expert, r_lo + rows_per_block);
    const int64_t ebytes = (int64_t)rows_per_expert * row_bytes;
    const __amdgpu_buffer_rsrc_t rs0 = wave_buffer(w0 + (int64_t)e * ebytes, (uint32_t)ebytes);
    const __amdgpu_buffer_rsrc_t rs1 = wave_buffer((GATED ? w1 : w0) + (int64_t)e * ebytes, (uint32_t)ebytes);
    for (int g0 = 0; g0 < cnt; g0 += group) {
        const int gn = min(group, cnt - g0);
        __syncthreads();  // the previous group's vectors are no longer read
        for (int i = threadIdx.x; i < gn * c4; i += 256) {
            const int q = i / c4, j = 4 * (i - q * c4);
            const int p = pairs[p0 + g0 + q];
            const float4 v = *reinterpret_cast<const float4 *>(vec + (int64_t)(by_pair ? p : p / top_k) * vec_stride + j);
            *reinterpret_cast<float4 *>(xs + q * rstride + goff(j >> 5) + (j & 31)) = v;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < 2 * gn * ng; i += 256) {  // the 16-element sums
            const int qg = i >> 1, q = qg / ng, g = qg - q * ng;
            float *xb = xs + q * rstride + goff(g);
            float t = 0.0f;
            for (int k = 0; k < 16; k++) t += xb[16 * (i & 1) + k];
            xb[32 + (i & 1)] = t;
        }
        __syncthreads();
        for (int r0 = r_lo + wave * RPW; r0 < r_hi; r0 += 4 * RPW) {
            const int r = r0 + rsub;
            const bool live = r < r_hi;
            const uint32_t row_off = live ? (uint32_t)((int64_t)r * row_bytes) : 0u;
            // One route at a time, gate then up (later routes re-read the
            // rows from the caches).
#pragma unroll 1
            for (int q = 0; q < gn; q++) {
                float a = 0.0f, u = 0.0f;
#pragma unroll 1
                for (int b = sub; b < nsb; b += LPR) {
                    if (!live) break;
                    const uint32_t off = row_off + (uint32_t)(b * kSB);
                    const float *xg = xs + q * rstride + 292 * b;
                    // gate and up dwords in flight together, then each contracted
                    KqRaw<T> raw0, raw1;
                    kq_load<T>(rs0, off, raw0);
                    if constexpr (GATED) kq_load<T>(rs1, off, raw1);
                    a += kq_dot<T>(raw0, off & 3u, xg);
                    if constexpr (GATED) u += kq_dot<T>(raw1, off & 3u, xg);
                }
                float v = group_sum<LPR>(a);
                if constexpr (GATED) {
                    const float uu = group_sum<LPR>(u);
                    v = v / (1.0f + expf(-v)) * uu;  // silu(gate) * up
                }
                if (sub == 0 && live) out[(int64_t)pairs[p0 + g0 + q] * out_stride + r] = v;
            }
        }
    }
}

// Lanes per row for rows of nsb superblocks: one superblock per lane (up
// to 64 lanes), so a row's loads are one round trip.
inline int kq_lanes_per_row(int nsb) {
    int l = 1;
    while (l < 64 && l < nsb) l *= 2;
    return l;
}

template <int T, bool GATED>
hipError_t launch_kq_expert(dim3 grid, size_t lds, hipStream_t stream, const uint8_t *w0, const uint8_t *w1,
                            int64_t row_bytes, int cols, int rows_per_expert, int rows_per_block,
                            const float *vec, int64_t vec_stride, int by_pair, int top_k, const int32_t *meta,
                            int E, int P, int group, float *out, int64_t out_stride) {
    const int lpr = kq_lanes_per_row(cols / 256);
#define GOLLEK_KQ_LAUNCH(L)                                                                              \
    hipLaunchKernelGGL((moe_kq_expert_kernel<T, GATED, L>), grid, dim3(256), lds, stream, w0, w1, row_bytes, \
                       cols, rows_per_expert, rows_per_block, vec, vec_stride, by_pair, top_k, meta, E, P, \
                       group, out, out_stride)
    if (lpr == 1) GOLLEK_KQ_LAUNCH(1);
    else if (lpr == 2) GOLLEK_KQ_LAUNCH(2);
    else if (lpr == 4) GOLLEK_KQ_LAUNCH(4);
    else if (lpr == 8) GOLLEK_KQ_LAUNCH(8);
    else if (lpr == 16) GOLLEK_KQ_LAUNCH(16);
    else if (lpr == 32) GOLLEK_KQ_LAUNCH(32);
    else GOLLEK_KQ_LAUNCH(64);
#undef GOLLEK_KQ_LAUNCH
    return hipGetLastError();
}

// Lanes per row for rows of nb blocks: about four blocks per lane, 8 .. 64.
inline int q32_lanes_per_row(int nb) {
    int l = 8;
    while (l < 64 && 4 * l < nb) l *= 2;
    return l;
}

template <int T, bool GATED>
hipError_t launch_q32_expert(dim3 grid, size_t lds, hipStream_t stream, const uint8_t *w0, const uint8_t *w1,
                             int64_t row_bytes, int cols, int rows_per_expert, int rows_per_block,
                             const float *vec, int64_t vec_stride, int by_pair, int top_k, const int32_t *meta,
                             int E, int P, int group, float *out, int64_t out_stride) {
    const int lpr = q32_lanes_per_row(cols / 32);
#define GOLLEK_Q32_LAUNCH(L)                                                                              \
    hipLaunchKernelGGL((moe_q32_expert_kernel<T, GATED, L>), grid, dim3(256), lds, stream, w0, w1, row_bytes, \
                       cols, rows_per_expert, rows_per_block, vec, vec_stride, by_pair, top_k, meta, E, P,  \
                       group, out, out_stride)
    if (lpr == 8) GOLLEK_Q32_LAUNCH(8);
    else if (lpr == 16) GOLLEK_Q32_LAUNCH(16);
    else if (lpr == 32) GOLLEK_Q32_LAUNCH(32);
    else GOLLEK_Q32_LAUNCH(64);
#undef GOLLEK_Q32_LAUNCH
    return hipGetLastError();
}

namespace {

template <bool GATED>
hipError_t launch_expert(int nsb, const uint8_t *w0, const uint8_t *w1, int64_t row_bytes,
                         int rows_per_expert, int rows_per_block, const uint8_t *digits,
                         int64_t digit_stride, int by_pair, int top_k, const int32_t *meta, int E,
                         int P, float *out, int64_t out_stride, hipStream_t stream) {
    const dim3 grid((rows_per_expert + rows_per_block - 1) / rows_per_block, E);
    const size_t lds = (size_t)kMoeTokensPerPass * digit_stride;
#define GOLLEK_MOE_LAUNCH(L)                                                                     \
    hipLaunchKernelGGL((moe_expert_kernel<L, GATED, 2>), grid, dim3(256), lds, stream, w0, w1,   \
                       row_bytes, nsb, rows_per_expert, rows_per_block, digits, digit_stride,    \
                       by_pair, top_k, meta, E, P, out, out_stride)
    if (nsb > 8) GOLLEK_MOE_LAUNCH(64);
    else if (nsb > 4) GOLLEK_MOE_LAUNCH(32);
    else if (nsb > 2) GOLLEK_MOE_LAUNCH(16);
    else if (nsb > 1) GOLLEK_MOE_LAUNCH(8);
    else GOLLEK_MOE_LAUNCH(4);
#undef GOLLEK_MOE_LAUNCH
    return hipGetLastError();
}

}  // namespace

hipError_t launch_moe_route(const int32_t *ids, const float *wts, int P, int E, int tiles0,
                            int tiles1, int32_t *meta, hipStream_t stream) {
    // The routes' keys stay in LDS for the scatter when they fit the default
    // 64 KB (the scatter otherwise reloads them, one round trip per 64).
    const size_t base = 2 * (size_t)E * sizeof(int32_t);
    const int keys_in_lds = base + (size_t)P * sizeof(int32_t) <= 65536 ? 1 : 0;
    hipLaunchKernelGGL(moe_route_kernel, dim3(1), dim3(256), base + (keys_in_lds ? (size_t)P * sizeof(int32_t) : 0),
                       stream, ids, wts, P, E, tiles0, tiles1, meta, keys_in_lds);
    return hipGetLastError();
}

hipError_t launch_moe_combine(const int32_t *ids, const float *wts, const float *ypair, int T,
                              int top_k, int H, int E, float *out, hipStream_t stream) {
    const int64_t total = (int64_t)T * H;
    hipLaunchKernelGGL(moe_combine_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       stream, ids, wts, ypair, T, top_k, H, E, out);
    return hipGetLastError();
}

MoeSharedLayout moe_shared_layout(int64_t tokens, int64_t hidden, int64_t inter) {
    auto up256 = [](size_t v) { return (v + 255) & ~(size_t)255; };
    MoeSharedLayout L;
    L.y = 0;
    L.ids = up256((size_t)(tokens * hidden) * 4);
    L.wts = L.ids + up256((size_t)tokens * 4);
    L.ffn = L.wts + up256((size_t)tokens * 4);
    L.total = L.ffn + moe_layout(tokens, 1, hidden, inter, 1).total;
    return L;
}

hipError_t launch_moe_shared(int gate_type, int up_type, int down_type, const uint8_t *gate, const uint8_t *up,
                             const uint8_t *down, int64_t gate_row_bytes, int64_t up_row_bytes,
                             int64_t down_row_bytes, int H, int I, const float *x, const float *gate_inp, int T,
                             float *out, uint8_t *ws, hipStream_t stream) {
    const MoeSharedLayout L = moe_shared_layout(T, H, I);
    float *y = reinterpret_cast<float *>(ws + L.y);
    int32_t *ids = reinterpret_cast<int32_t *>(ws + L.ids);
    float *wts = reinterpret_cast<float *>(ws + L.wts);
    hipLaunchKernelGGL(moe_shared_routes_kernel, dim3((unsigned)((T + 255) / 256)), dim3(256), 0, stream, ids, wts,
                       T);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    // y[t] = 0 + 1 * ffn(x_t): the expert's output exactly
    e = launch_moe(gate_type, up_type, down_type, gate, up, down, gate_row_bytes, up_row_bytes, down_row_bytes, 1,
                   H, I, x, ids, wts, T, 1, y, ws + L.ffn, stream);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(moe_shared_add_kernel, dim3((unsigned)T), dim3(256), 0, stream, x, gate_inp, y, H, out);
    return hipGetLastError();
}

// Expert FFN on the generic kernels: routing, gate/up (h = silu(g) u into
// the workspace's h), down (per-route rows into ypair), route-order combine.
hipError_t launch_moe_generic(int gate_type, int up_type, int down_type, const uint8_t *gate,
                              const uint8_t *up, const uint8_t *down, int64_t gate_row_bytes,
                              int64_t up_row_bytes, int64_t down_row_bytes, int E, int H, int I,
                              const float *x, const int32_t *ids, const float *wts, int T, int top_k,
                              float *out, uint8_t *ws, hipStream_t stream) {
    const MoeLayout L = moe_layout(T, top_k, H, I, E);
    const int P = T * top_k;
    int32_t *meta = reinterpret_cast<int32_t *>(ws + L.meta);
    hipError_t err = launch_moe_route(ids, wts, P, E, 0, 0, meta, stream);
    if (err != hipSuccess) return err;
    float *h = reinterpret_cast<float *>(ws + L.h);
    float *ypair = reinterpret_cast<float *>(ws + L.ypair);
    constexpr int kRows = 64;
    // Q8_0 / Q4_0 passes: the route vectors of a group in LDS (at most 96 KiB).
    auto q32_group = [](int cols) {
        const int g = (96 * 1024) / ((cols / 32) * 144);
        return g < kQ32Group ? g : kQ32Group;
    };
    // K-quant passes: 36 floats per 32 elements and 4 more per superblock.
    auto kq_route_bytes = [](int cols) { return (size_t)((cols / 32) * 36 + (cols / 256) * 4) * 4; };
    auto kq_group = [&](int cols) {
        const int g = (int)((96 * 1024) / kq_route_bytes(cols));
        return g < kQ32Group ? g : kQ32Group;
    };
    const bool x_aligned = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
    const int g_gu = q32_group(H), g_dn = q32_group(I);
    if (gate_type == up_type && (gate_type == kQ8_0 || gate_type == kQ4_0) && x_aligned && g_gu > 0 &&
        gate_row_bytes == up_row_bytes && (int64_t)I * gate_row_bytes < ((int64_t)1 << 31)) {
        const size_t lds = (size_t)g_gu * (H / 32) * 144;
        const dim3 grid((I + kRows - 1) / kRows, E);
        if (gate_type == kQ8_0)
            err = launch_q32_expert<kQ8_0, true>(grid, lds, stream, gate, up, gate_row_bytes, H, I, kRows, x, (int64_t)H, 0,
                                           top_k, meta, E, P, g_gu, h, (int64_t)I);
        else
            err = launch_q32_expert<kQ4_0, true>(grid, lds, stream, gate, up, gate_row_bytes, H, I, kRows, x, (int64_t)H, 0,
                                           top_k, meta, E, P, g_gu, h, (int64_t)I);
    } else if (gate_type == up_type && (gate_type == kQ4_K || gate_type == kQ5_K || gate_type == kQ6_K) &&
               x_aligned && kq_group(H) > 0 && H % 256 == 0 && gate_row_bytes == up_row_bytes &&
               (int64_t)I * gate_row_bytes < ((int64_t)1 << 31)) {
        const int g_kq = kq_group(H);
        const size_t lds = (size_t)g_kq * kq_route_bytes(H);
        const dim3 grid((I + kRows - 1) / kRows, E);
        if (gate_type == kQ4_K)
            err = launch_kq_expert<kQ4_K, true>(grid, lds, stream, gate, up, gate_row_bytes, H, I, kRows, x, (int64_t)H,
                                                0, top_k, meta, E, P, g_kq, h, (int64_t)I);
        else if (gate_type == kQ5_K)
            err = launch_kq_expert<kQ5_K, true>(grid, lds, stream, gate, up, gate_row_bytes, H, I, kRows, x, (int64_t)H,
                                                0, top_k, meta, E, P, g_kq, h, (int64_t)I);
        else
            err = launch_kq_expert<kQ6_K, true>(grid, lds, stream, gate, up, gate_row_bytes, H, I, kRows, x, (int64_t)H,
                                                0, top_k, meta, E, P, g_kq, h, (int64_t)I);
    } else {
        hipLaunchKernelGGL(moe_generic_expert_kernel<true>, dim3((I + kRows - 1) / kRows, E), dim3(256), 0, stream,
                           gate_type, up_type, gate, up, gate_row_bytes, up_row_bytes, H, I, kRows, x, (int64_t)H, 0,
                           top_k, meta, E, P, h, (int64_t)I);
        err = hipGetLastError();
    }
    if (err != hipSuccess) return err;
    if ((down_type == kQ8_0 || down_type == kQ4_0) && g_dn > 0 &&
        (int64_t)H * down_row_bytes < ((int64_t)1 << 31)) {
        const size_t lds = (size_t)g_dn * (I / 32) * 144;
        const dim3 grid((H + kRows - 1) / kRows, E);
        if (down_type == kQ8_0)
            err = launch_q32_expert<kQ8_0, false>(grid, lds, stream, down, down, down_row_bytes, I, H, kRows, h, (int64_t)I,
                                            1, top_k, meta, E, P, g_dn, ypair, (int64_t)H);
        else
            err = launch_q32_expert<kQ4_0, false>(grid, lds, stream, down, down, down_row_bytes, I, H, kRows, h, (int64_t)I,
                                            1, top_k, meta, E, P, g_dn, ypair, (int64_t)H);
    } else if ((down_type == kQ4_K || down_type == kQ5_K || down_type == kQ6_K) && kq_group(I) > 0 &&
               I % 256 == 0 && (int64_t)H * down_row_bytes < ((int64_t)1 << 31)) {
        const int g_kq = kq_group(I);
        const size_t lds = (size_t)g_kq * kq_route_bytes(I);
        const dim3 grid((H + kRows - 1) / kRows, E);
        if (down_type == kQ4_K)
            err = launch_kq_expert<kQ4_K, false>(grid, lds, stream, down, down, down_row_bytes, I, H, kRows, h,
                                                 (int64_t)I, 1, top_k, meta, E, P, g_kq, ypair, (int64_t)H);
        else if (down_type == kQ5_K)
            err = launch_kq_expert<kQ5_K, false>(grid, lds, stream, down, down, down_row_bytes, I, H, kRows, h,
                                                 (int64_t)I, 1, top_k, meta, E, P, g_kq, ypair, (int64_t)H);
        else
            err = launch_kq_expert<kQ6_K, false>(grid, lds, stream, down, down, down_row_bytes, I, H, kRows, h,
                                                 (int64_t)I, 1, top_k, meta, E, P, g_kq, ypair, (int64_t)H);
    } else {
        hipLaunchKernelGGL(moe_generic_expert_kernel<false>, dim3((H + kRows - 1) / kRows, E), dim3(256), 0, stream,
                           down_type, down_type, down, down, down_row_bytes, down_row_bytes, I, H, kRows, h,
                           (int64_t)I, 1, top_k, meta, E, P, ypair, (int64_t)H);
        err = hipGetLastError();
    }
    if (err != hipSuccess) return err;
    return launch_moe_combine(ids, wts, ypair, T, top_k, H, E, out, stream);
}

hipError_t launch_moe(int gate_type, int up_type, int down_type, const uint8_t *gate, const uint8_t *up,
                      const uint8_t *down, int64_t gate_row_bytes, int64_t up_row_bytes,
                      int64_t down_row_bytes, int E, int H, int I, const float *x, const int32_t *ids,
                      const float *wts, int T, int top_k, float *out, uint8_t *ws, hipStream_t stream) {
    const bool aligned = ((reinterpret_cast<uintptr_t>(gate) | reinterpret_cast<uintptr_t>(up) |
                           reinterpret_cast<uintptr_t>(down) | reinterpret_cast<uintptr_t>(x)) & 15u) == 0;
    const bool q4k_gu = gate_type == kQ4_K && up_type == kQ4_K;
    // More routes than the matrix-core passes route in LDS (prefill): token
    // slices of at most kMoeMfmaMaxRoutes / top_k tokens, one after another on
    // the stream, when a slice takes those passes (a token's output depends on
    // its own routes only, so the results do not change).
    const int tslice = kMoeMfmaMaxRoutes / top_k;
    if (aligned && (int64_t)T * top_k > kMoeMfmaMaxRoutes && tslice >= 1 && tuning().moe_variant != 1 &&
        ((gate_type == up_type && moe_kq_mfma_supported(gate_type, down_type, E, H, I, tslice, top_k, x)) ||
         (gate_type == kQ4_0 && up_type == kQ4_0 && down_type == kQ4_0 &&
          moe_q40_mfma_supported(E, H, I, tslice * top_k, x)))) {
        for (int t0 = 0; t0 < T; t0 += tslice) {
            const int tn = T - t0 < tslice ? T - t0 : tslice;
            const hipError_t e = launch_moe(gate_type, up_type, down_type, gate, up, down, gate_row_bytes,
                                            up_row_bytes, down_row_bytes, E, H, I, x + (int64_t)t0 * H,
                                            ids + (int64_t)t0 * top_k, wts + (int64_t)t0 * top_k, tn, top_k,
                                            out + (int64_t)t0 * H, ws, stream);
            if (e != hipSuccess) return e;
        }
        return hipSuccess;
    }
    // Q4_K or Q5_K gate / up with the down types the matrix-core passes take.
    if (aligned && gate_type == up_type && tuning().moe_variant != 1 &&
        moe_kq_mfma_supported(gate_type, down_type, E, H, I, T, top_k, x))
        return launch_moe_kq_mfma(gate_type, down_type, gate, up, down, E, H, I, x, ids, wts, T, top_k, out, ws,
                                  stream);
    // All Q4_0 (hidden up to 2048): the matrix-core passes with Q4_0 rows.
    if (aligned && gate_type == kQ4_0 && up_type == kQ4_0 && down_type == kQ4_0 && tuning().moe_variant != 1 &&
        moe_q40_mfma_supported(E, H, I, T * top_k, x))
        return launch_moe_q40_mfma(gate, up, down, E, H, I, x, ids, wts, T, top_k, out, ws, stream);
    // All Q4_K up to hidden / inter 4096: the v_dot4 passes.
    if (aligned && q4k_gu && down_type == kQ4_K && H % kQK == 0 && I % kQK == 0 && H <= 4096 && I <= 4096)
        return launch_moe_q4k_dot4(gate, up, down, gate_row_bytes, down_row_bytes, E, H, I, x, ids, wts, T,
                                   top_k, out, ws, stream);
    return launch_moe_generic(gate_type, up_type, down_type, gate, up, down, gate_row_bytes, up_row_bytes,
                              down_row_bytes, E, H, I, x, ids, wts, T, top_k, out, ws, stream);
}

hipError_t launch_moe_q4k_dot4(const uint8_t *gate, const uint8_t *up, const uint8_t *down,
                               int64_t gate_row_bytes, int64_t down_row_bytes, int E, int H, int I,
                               const float *x, const int32_t *ids, const float *wts, int T, int top_k,
                               float *out, uint8_t *ws, hipStream_t stream) {
    const MoeLayout L = moe_layout(T, top_k, H, I, E);
    const int P = T * top_k;
    int32_t *meta = reinterpret_cast<int32_t *>(ws + L.meta);
    hipError_t rerr = launch_moe_route(ids, wts, P, E, 0, 0, meta, stream);
    if (rerr != hipSuccess) return rerr;
    hipLaunchKernelGGL(moe_digits_kernel, dim3(T), dim3(256), 0, stream, x, H, (int64_t)H,
                       ws + L.xdig, (int64_t)L.xdig_stride);
    hipError_t err = launch_expert<true>(H / kQK, gate, up, gate_row_bytes, I, 64, ws + L.xdig,
                                         (int64_t)L.xdig_stride, 0, top_k, meta, E, P,
                                         reinterpret_cast<float *>(ws + L.h), I, stream);
    if (err != hipSuccess) return err;
    hipLaunchKernelGGL(moe_digits_kernel, dim3(P), dim3(256), 0, stream,
                       reinterpret_cast<const float *>(ws + L.h), I, (int64_t)I, ws + L.hdig,
                       (int64_t)L.hdig_stride);
    err = launch_expert<false>(I / kQK, down, nullptr, down_row_bytes, H, 128, ws + L.hdig,
                               (int64_t)L.hdig_stride, 1, top_k, meta, E, P,
                               reinterpret_cast<float *>(ws + L.ypair), H, stream);
    if (err != hipSuccess) return err;
    return launch_moe_combine(ids, wts, reinterpret_cast<const float *>(ws + L.ypair), T, top_k, H,
                              E, out, stream);
}

}  // namespace gollek
