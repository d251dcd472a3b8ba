// gguf_moe_router.hip -- MoE router: per token, router logits -> expert
// probabilities (softmax or sigmoid) -> the top_k experts -> weights
// renormalised over the chosen ones.
//
// Follows SFE/generation/moe/MoeForwardPass.java (SFE/ = runner/safetensor/
// gollek-safetensor-engine/src/main/java/tech/kayys/gollek/safetensor/engine/)
// with its rounding:
//   * sigmoid (:178-181): p = 1.0f / (1.0f + (float)exp(-l)), exp in double;
//   * softmax (:182-197): max over the row (Math.max: NaN wins), then
//     p = (float)exp(l - max) with the difference in float and exp in double,
//     the float sum in expert order, then p / sum;
//   * top-k (selectTopK :286-306): experts in descending Float.compare order,
//     ties (equal bits; every NaN counts as one value above +inf) in index
//     order (a stable sort); weights are the chosen probabilities divided by
//     their float sum, taken in rank order, when that sum is > 0.  Ranks past
//     the expert count keep id 0 and weight 0.
//
// One 256-thread workgroup per token.  Each thread owns experts e = tid,
// tid + 256, ...; the two order-dependent float sums run in one lane of wave
// 0 over values the wave loaded together (E and top_k adds, one lane read
// each), everything else is parallel.  A thread finds the rank of its expert
// by counting, over all experts (four keys per LDS read), the keys above its
// own plus the equal keys at lower indices: the position a stable
// descending sort gives it.
#include <hip/hip_runtime.h>

#include "gguf_kernels.hpp"

namespace gollek {
namespace {

constexpr int kRouterThreads = 256;

// Java's Float.compare order as a signed integer: floatToIntBits (every NaN
// becomes 0x7FC00000), then negative floats reflected so that integer order
// is float order, -0.0 below +0.0 and NaN above +inf.
__device__ inline int order_key(float v) {
    int b = v != v ? 0x7FC00000 : __float_as_int(v);
    return b >= 0 ? b : b ^ 0x7FFFFFFF;
}

// Math.max: NaN if either is NaN, +0.0 over -0.0.
__device__ inline float java_max(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    if (a == 0.0f && b == 0.0f) return __float_as_int(a) == 0 ? a : b;
    return a > b ? a : b;
}

// Sum of v[0, n) in index order (s = ((0 + v0) + v1) + ...), v in LDS: wave 0
// loads 64 values at a time and one lane adds them in order.  Every lane of
// wave 0 calls this; the sum is returned in all of them.
__device__ inline float ordered_sum(const float *v, int n, int lane) {
#pragma clang fp contract(off)
    float s = 0.0f;
    for (int base = 0; base < n; base += 64) {
        const float mine = base + lane < n ? v[base + lane] : 0.0f;
        const int m = n - base < 64 ? n - base : 64;
        for (int j = 0; j < m; j++) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), j));
    }
    return s;
}

__global__ __launch_bounds__(kRouterThreads) void moe_topk_kernel(
    const float *__restrict__ logits, int E, int K, int sigmoid, int32_t *__restrict__ ids,
    float *__restrict__ wts) {
#pragma clang fp contract(off)
    // key[E4] (as int, padded to a multiple of 4 with keys that count for
    // nothing), p[E], sel[K], red[kRouterThreads / 64]
    extern __shared__ __attribute__((aligned(16))) int sh[];
    const int E4 = (E + 3) & ~3;
    int *key = sh;
    float *p = reinterpret_cast<float *>(sh + E4);
    int *sel = reinterpret_cast<int *>(p + E);
    float *red = reinterpret_cast<float *>(sel + K);
    __shared__ float s_max, s_sum;
    const int t = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const float *row = logits + (size_t)t * E;

    if (sigmoid) {
        for (int e = tid; e < E; e += kRouterThreads) {
            const float l = row[e];
            p[e] = 1.0f / (1.0f + (float)exp((double)(-l)));
        }
    } else {
        float m = -__builtin_inff();
        for (int e = tid; e < E; e += kRouterThreads) m = java_max(m, row[e]);
        for (int off = 32; off > 0; off >>= 1) m = java_max(m, __shfl_xor(m, off));
        if ((tid & 63) == 0) red[tid >> 6] = m;
        __syncthreads();
        if (tid == 0) {
            float mm = red[0];
            for (int w = 1; w < kRouterThreads / 64; w++) mm = java_max(mm, red[w]);
            s_max = mm;
        }
        __syncthreads();
        const float mx = s_max;
        for (int e = tid; e < E; e += kRouterThreads) p[e] = (float)exp((double)(row[e] - mx));
        __syncthreads();
        if (tid < 64) {
            const float s = ordered_sum(p, E, lane);
            if (tid == 0) s_sum = s;
        }
        __syncthreads();
        const float s = s_sum;
        for (int e = tid; e < E; e += kRouterThreads) p[e] = p[e] / s;
    }
    for (int k = tid; k < K; k += kRouterThreads) sel[k] = -1;
    __syncthreads();
    // INT_MIN is below every key order_key gives (-inf maps above it) and
    // equal to none: the padding adds nothing to a rank.
    for (int e = tid; e < E4; e += kRouterThreads) key[e] = e < E ? order_key(p[e]) : INT_MIN;
    __syncthreads();
    // Keys above key[e] plus equal keys below e, over keys [j0, j1).
    auto count = [&](int e, int j0, int j1) {
        const int me = key[e];
        int rank = 0;
#pragma unroll 4
        for (int j = j0; j < j1; j += 4) {
            const int4 k4 = *reinterpret_cast<const int4 *>(key + j);
            rank += (k4.x > me) | ((k4.x == me) & (j < e));
            rank += (k4.y > me) | ((k4.y == me) & (j + 1 < e));
            rank += (k4.z > me) | ((k4.z == me) & (j + 2 < e));
            rank += (k4.w > me) | ((k4.w == me) & (j + 3 < e));
        }
        return rank;
    };
    // Up to 8 threads per expert when the experts leave threads idle, each
    // counting one span of the keys; the spans' counts are added in LDS.
    int tpe = 1;
    while (tpe < 8 && 2 * tpe * E <= kRouterThreads) tpe *= 2;  // uniform
    if (tpe == 1) {
        for (int e = tid; e < E; e += kRouterThreads) {
            const int rank = count(e, 0, E4);
            if (rank < K) sel[rank] = e;
        }
    } else {
        __shared__ int prank[kRouterThreads];
        const int span = (E4 / tpe + 3) & ~3;
        if (tid < tpe * E) {
            const int e = tid % E, part = tid / E;
            const int j0 = part * span, j1 = j0 + span < E4 ? j0 + span : E4;
            prank[tid] = count(e, j0, j1);
        }
        __syncthreads();
        if (tid < E) {
            int rank = 0;
            for (int q = 0; q < tpe; q++) rank += prank[q * E + tid];
            if (rank < K) sel[rank] = tid;
        }
    }
    __syncthreads();
    if (tid < 64) {
        // chosen probabilities of ranks k < n, summed in rank order
        const int n = K < E ? K : E;
        float s = 0.0f;
        for (int base = 0; base < n; base += 64) {
            const float mine = base + lane < n ? p[sel[base + lane]] : 0.0f;
            const int m = n - base < 64 ? n - base : 64;
            for (int j = 0; j < m; j++) s += __int_as_float(__builtin_amdgcn_readlane(__float_as_int(mine), j));
        }
        for (int k = lane; k < K; k += 64) {
            const bool have = k < n;
            float w = have ? p[sel[k]] : 0.0f;
            if (s > 0.0f) w = w / s;
            ids[(size_t)t * K + k] = have ? sel[k] : 0;
            wts[(size_t)t * K + k] = w;
        }
    }
}

}  // namespace

size_t moe_topk_lds_bytes(int E, int K) {
    return (size_t)((E + 3) & ~3) * 4 + (size_t)E * 4 + (size_t)K * 4 + (kRouterThreads / 64) * 4;
}

hipError_t launch_moe_topk(const float *logits, int T, int E, int K, int sigmoid, int32_t *ids,
                           float *wts, hipStream_t stream) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(moe_topk_kernel, dim3(T), dim3(kRouterThreads), moe_topk_lds_bytes(E, K),
                       stream, logits, E, K, sigmoid, ids, wts);
    return hipGetLastError();
}

}  // namespace gollek
