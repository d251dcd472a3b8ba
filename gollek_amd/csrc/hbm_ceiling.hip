// hbm_ceiling.hip -- measurement kernels for bench.py --ceilings (built into
// libgollek_ceiling.so, not part of the product library or its C ABI).
//
// They give the device's attainable figures for the rooflines of the GEMV
// kernels: how long a single launch takes to stream B bytes from HBM with
// the plainest possible kernel, for several grids and load kinds, and how
// long an empty launch of the same grid takes (the per-launch floor of a
// stream of dependent launches).
//
//   kind 0: global_load_dwordx4 into registers, nontemporal, every load of a
//           wave issued before the first is used;
//   kind 1: the same with the default cache policy;
//   kind 2: buffer->LDS loads of 1 KB per wave instruction, nontemporal,
//           every load issued up front, one wait;
//   kind 3: an empty kernel of the same grid.
//
// Each wave reads one contiguous chunk of ceil(bytes / 16 / waves) 16-byte
// items.  Register kinds fold the data into one dword per thread (written to
// `out`, which must hold blocks * threads dwords) so no load is dead.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void *lds_ptr;

template <int L, bool NT>
__global__ void read_reg_kernel(const u32x4 *__restrict__ p, int64_t n16, int64_t per_wave,
                                uint32_t *__restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t b = wave * per_wave;
    const int64_t e = b + per_wave < n16 ? b + per_wave : n16;
    u32x4 v[L];
#pragma unroll
    for (int i = 0; i < L; i++) {
        const int64_t j = b + lane + 64 * i;
        if (j < e) v[i] = NT ? __builtin_nontemporal_load(p + j) : p[j];
        else v[i] = u32x4{0u, 0u, 0u, 0u};
    }
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < L; i++) acc ^= v[i].x ^ v[i].y ^ v[i].z ^ v[i].w;
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = acc;
}

template <int L>
__global__ void read_lds_kernel(const uint8_t *__restrict__ p, int64_t bytes, int64_t per_wave16,
                                uint32_t *__restrict__ out) {
    extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
    const int lane = threadIdx.x & 63;
    const int wib = threadIdx.x >> 6;
    const int64_t wave = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) >> 6;
    const int64_t b = wave * per_wave16 * 16;  // first byte of the wave's chunk
    int64_t len = bytes - b;
    if (len > per_wave16 * 16) len = per_wave16 * 16;
    if (len < 0) len = 0;
    // The descriptor covers the wave's chunk only; offsets past it read zeros.
    const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t *>(p) + (b < bytes ? b : 0), 0, (int)len, 0x00020000);
    uint8_t *mine = lds + (size_t)wib * L * 1024;
#pragma unroll
    for (int i = 0; i < L; i++)
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr)(mine + 1024 * i), 16,
                                                 (uint32_t)(1024 * i + 16 * lane), 0, 0, 2);
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    out[(int64_t)blockIdx.x * blockDim.x + threadIdx.x] = reinterpret_cast<const uint32_t *>(mine)[lane];
}

__global__ void empty_kernel(uint32_t *__restrict__ out) {
    if (blockIdx.x == 0x7FFFFFFF) out[threadIdx.x] = 0;  // never true; keeps the argument live
}

template <int L>
hipError_t launch_reg(bool nt, const u32x4 *p, int64_t n16, int64_t pw, uint32_t *o, int blocks,
                      int threads, hipStream_t s) {
    if (nt) hipLaunchKernelGGL((read_reg_kernel<L, true>), dim3(blocks), dim3(threads), 0, s, p, n16, pw, o);
    else hipLaunchKernelGGL((read_reg_kernel<L, false>), dim3(blocks), dim3(threads), 0, s, p, n16, pw, o);
    return hipGetLastError();
}

}  // namespace

extern "C" {

// Loads a lane issues for `bytes` over blocks * waves_per_block waves
// (kinds 0-2), or -1 when the kind cannot run that shape.
int64_t gollek_ceiling_loads_per_lane(int32_t kind, int64_t bytes, int32_t blocks,
                                      int32_t waves_per_block) {
    const int64_t waves = (int64_t)blocks * waves_per_block;
    if (waves <= 0 || bytes < 0) return -1;
    const int64_t pw = ((bytes + 15) / 16 + waves - 1) / waves;
    const int64_t L = (pw + 63) / 64;
    if (kind == 2) {
        // dynamic LDS of the kernel instance (<= 64 KB without an attribute)
        const int64_t t = L <= 4 ? 4 : L <= 8 ? 8 : L <= 9 ? 9 : 16;
        return (L <= 16 && waves_per_block * t <= 64) ? L : -1;
    }
    if (kind == 0 || kind == 1) return L <= 32 ? L : -1;
    return 0;
}

// One launch of kind `kind` over `bytes` bytes at `p` (16-byte aligned) on
// `stream`; returns a hipError_t (-1 for a shape the kind cannot run).
int32_t gollek_ceiling_launch(int32_t kind, const void *p, int64_t bytes, void *out, int32_t blocks,
                              int32_t waves_per_block, void *stream) {
    hipStream_t s = (hipStream_t)stream;
    uint32_t *o = (uint32_t *)out;
    const int threads = 64 * waves_per_block;
    const int64_t L = gollek_ceiling_loads_per_lane(kind, bytes, blocks, waves_per_block);
    if (L < 0 || threads > 1024) return -1;
    const int64_t waves = (int64_t)blocks * waves_per_block;
    const int64_t n16 = bytes / 16;
    const int64_t pw = (n16 + waves - 1) / waves;
    if (kind == 3) {
        hipLaunchKernelGGL(empty_kernel, dim3(blocks), dim3(threads), 0, s, o);
        return (int32_t)hipGetLastError();
    }
    if (kind == 2) {
        const size_t lds = (size_t)waves_per_block * 1024 * (L <= 4 ? 4 : L <= 8 ? 8 : L <= 9 ? 9 : 16);
        const uint8_t *b = (const uint8_t *)p;
        if (L <= 4) hipLaunchKernelGGL((read_lds_kernel<4>), dim3(blocks), dim3(threads), lds, s, b, bytes, pw, o);
        else if (L <= 8) hipLaunchKernelGGL((read_lds_kernel<8>), dim3(blocks), dim3(threads), lds, s, b, bytes, pw, o);
        else if (L <= 9) hipLaunchKernelGGL((read_lds_kernel<9>), dim3(blocks), dim3(threads), lds, s, b, bytes, pw, o);
        else hipLaunchKernelGGL((read_lds_kernel<16>), dim3(blocks), dim3(threads), lds, s, b, bytes, pw, o);
        return (int32_t)hipGetLastError();
    }
    const bool nt = kind == 0;
    const u32x4 *q = (const u32x4 *)p;
    if (L <= 4) return (int32_t)launch_reg<4>(nt, q, n16, pw, o, blocks, threads, s);
    if (L <= 8) return (int32_t)launch_reg<8>(nt, q, n16, pw, o, blocks, threads, s);
    if (L <= 16) return (int32_t)launch_reg<16>(nt, q, n16, pw, o, blocks, threads, s);
    return (int32_t)launch_reg<32>(nt, q, n16, pw, o, blocks, threads, s);
}

}  // extern "C"
