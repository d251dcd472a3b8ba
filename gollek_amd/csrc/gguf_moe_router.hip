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
// tid + 256, ...; the two order-dependent float sums run on one thread from
// LDS (E and top_k adds), everything else is parallel.  A thread finds the
// rank of its expert by counting, over all experts, the keys above its own
// plus the equal keys at lower indices: the position a stable descending
// sort gives it.
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

__global__ __launch_bounds__(kRouterThreads) void moe_topk_kernel(
    const float *__restrict__ logits, int E, int K, int sigmoid, int32_t *__restrict__ ids,
    float *__restrict__ wts) {
#pragma clang fp contract(off)
    extern __shared__ float sh[];  // p[E], key[E] (as int), sel[K], red[kRouterThreads / 64]
    float *p = sh;
    int *key = reinterpret_cast<int *>(sh + E);
    int *sel = key + E;
    float *red = reinterpret_cast<float *>(sel + K);
    __shared__ float s_max, s_sum;
    const int t = blockIdx.x, tid = threadIdx.x;
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
        if (tid == 0) {
            float s = 0.0f;
            for (int e = 0; e < E; e++) s += p[e];
            s_sum = s;
        }
        __syncthreads();
        const float s = s_sum;
        for (int e = tid; e < E; e += kRouterThreads) p[e] = p[e] / s;
    }
    for (int k = tid; k < K; k += kRouterThreads) sel[k] = -1;
    __syncthreads();
    for (int e = tid; e < E; e += kRouterThreads) key[e] = order_key(p[e]);
    __syncthreads();
    for (int e = tid; e < E; e += kRouterThreads) {
        const int me = key[e];
        int rank = 0;
        for (int j = 0; j < E; j++) {
            const int kj = key[j];
            rank += (kj > me) | ((kj == me) & (j < e));
        }
        if (rank < K) sel[rank] = e;
    }
    __syncthreads();
    if (tid == 0) {
        const int n = K < E ? K : E;
        float s = 0.0f;
        for (int k = 0; k < n; k++) s += p[sel[k]];
        for (int k = 0; k < K; k++) {
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
    return (size_t)E * 8 + (size_t)K * 4 + (kRouterThreads / 64) * 4;
}

hipError_t launch_moe_topk(const float *logits, int T, int E, int K, int sigmoid, int32_t *ids,
                           float *wts, hipStream_t stream) {
    if (T <= 0) return hipSuccess;
    hipLaunchKernelGGL(moe_topk_kernel, dim3(T), dim3(kRouterThreads), moe_topk_lds_bytes(E, K),
                       stream, logits, E, K, sigmoid, ids, wts);
    return hipGetLastError();
}

}  // namespace gollek
