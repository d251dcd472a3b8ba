// gguf_capi.hip -- the C ABI declared in include/gollek_hip.h.
//
// Validation mirrors the Java facade it replaces (RT/GgufTensorOps.java,
// RT/GgufMatVec.java, RT/GgufTensorShape.java:53-72, GC/core/GgmlType.java:
// 70-81; RT/ = runner/gguf/gollek-gguf-core/src/main/java/tech/kayys/gollek/
// gguf/runtime/) in both the checks and their order, so the Java adapter can
// rethrow the same exceptions with the same messages.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <atomic>
#include <cstring>
#include <mutex>
#include <new>
#include <string>

#include "gguf_kernels.hpp"
#include "gollek_hip.h"
#include "gollek_hip_testing.h"

struct gollek_hip_weight {
    int32_t type_id = 0;
    int64_t rows = 0, cols = 0, row_bytes = 0;
    int device = 0;
    uint8_t *data = nullptr;
    bool owned = false;
    std::mutex mu;                 // serialises the host-buffer entry points
    hipStream_t stream = nullptr;  // stream of the host-buffer entry points
    uint8_t *staging = nullptr;    // device staging for host x / y / dst
    size_t staging_bytes = 0;
    float *gemm_ws = nullptr;      // split-K partial tiles of the device GEMM entry
    size_t gemm_ws_bytes = 0;
    uint8_t *prep = nullptr;       // prepared column layout (gollek_hip_weight_prepare)
    int64_t prep_rows = 0;         // its rows per workgroup
    bool compact = false;          // GGUF bytes freed (gollek_hip_weight_compact): prep only
    uint8_t *ctmp = nullptr;       // device temporaries of a compact handle's _device entries
    size_t ctmp_bytes = 0;
    uint8_t *hstage = nullptr;     // pinned host staging for host x / y / dst
    size_t hstage_bytes = 0;
};

namespace {

constexpr int32_t kAbiVersion = 1 * 10000 + 0 * 100 + 0;
constexpr int64_t kRouterMaxExperts = 4096;  // router LDS: 8 B per expert + 4 B per rank

thread_local std::string g_last_error;
thread_local int32_t g_last_status = GOLLEK_HIP_OK;

int32_t fail(int32_t code, char *err, size_t err_len, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    try {
        g_last_error = buf;
    } catch (const std::bad_alloc &) {  // keep the status; the message is in err
        g_last_error.clear();
    }
    g_last_status = code;
    if (err != nullptr && err_len > 0) {
        size_t n = strlen(buf);
        if (n >= err_len) n = err_len - 1;
        memcpy(err, buf, n);
        err[n] = '\0';
    }
    return code;
}

void ok(char *err, size_t err_len) {
    g_last_error.clear();
    g_last_status = GOLLEK_HIP_OK;
    if (err != nullptr && err_len > 0) err[0] = '\0';
}

int32_t hip_fail(hipError_t e, const char *what, char *err, size_t err_len) {
    return fail(e == hipErrorOutOfMemory ? GOLLEK_HIP_ERR_NOMEM : GOLLEK_HIP_ERR_DEVICE, err,
                err_len, "%s failed: %s", what, hipGetErrorString(e));
}

const char *type_label(int32_t type_id) {
    switch (type_id) {
    case GOLLEK_HIP_Q4_0: return "Q4_0";
    case GOLLEK_HIP_Q8_0: return "Q8_0";
    case GOLLEK_HIP_Q4_K: return "Q4_K";
    case GOLLEK_HIP_Q5_K: return "Q5_K";
    case GOLLEK_HIP_Q6_K: return "Q6_K";
    default: return "?";
    }
}

// Elements and bytes per block (GC/core/GgmlType.java:11-24).
int block_size(int32_t type_id) { return type_id >= GOLLEK_HIP_Q4_K ? 256 : 32; }

int block_bytes(int32_t type_id) {
    switch (type_id) {
    case GOLLEK_HIP_Q4_0: return 18;
    case GOLLEK_HIP_Q8_0: return 34;
    case GOLLEK_HIP_Q4_K: return 144;
    case GOLLEK_HIP_Q5_K: return 176;
    default: return 210;  // Q6_K
    }
}

bool supported(int32_t type_id) {
    return type_id == GOLLEK_HIP_Q4_0 || type_id == GOLLEK_HIP_Q8_0 || type_id == GOLLEK_HIP_Q4_K ||
           type_id == GOLLEK_HIP_Q5_K || type_id == GOLLEK_HIP_Q6_K;
}

std::mutex g_init_mu;
int g_initialised_device = -1;

// Split-K scratch of gollek_hip_gemm_bf16_device_noalloc: a file-scope
// device array, so each GPU holds its own copy from module load until the
// process ends.  On the host, `scratch` only names that array; kernels get
// the per-device address hipGetSymbolAddress returns, resolved once per
// device (with the device current) when the library first sets it up.
constexpr size_t kGemmScratchBytes = (size_t)16 << 20;  // gemm_workspace_bytes < 16 MiB on 256 CUs
constexpr int kMaxDevices = 64;
static __device__ __align__(256) float scratch[kGemmScratchBytes / sizeof(float)];
std::atomic<float *> g_scratch_ptr[kMaxDevices];

// Makes `device` current on this thread, records its CU count and resolves
// its copy of the static GEMM scratch, once.
int32_t use_device(int device, char *err, size_t err_len) {
    hipError_t e = hipSetDevice(device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice", err, err_len);
    std::lock_guard<std::mutex> lock(g_init_mu);
    if (g_initialised_device != device) {
        int cus = 0;
        e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
        if (e != hipSuccess) return hip_fail(e, "hipDeviceGetAttribute", err, err_len);
        if (cus > 0) gollek::tuning().cu_count = cus;
        g_initialised_device = device;
    }
    if (device >= 0 && device < kMaxDevices && g_scratch_ptr[device].load() == nullptr) {
        void *ptr = nullptr;
        e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
        if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(scratch)", err, err_len);
        g_scratch_ptr[device].store(static_cast<float *>(ptr));
    }
    return GOLLEK_HIP_OK;
}

// GC/core/GgmlType.java:70-81 and RT/GgufTensorShape.java:185-198.
int32_t check_shape(int32_t type_id, int64_t rows, int64_t cols, int64_t row_bytes, char *err,
                    size_t err_len) {
    if (!supported(type_id))
        return fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len,
                    "Unsupported GGUF quantized matmul type id: %d", type_id);
    if (rows < 0 || cols <= 0)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Invalid matrix shape %lld x %lld",
                    (long long)rows, (long long)cols);
    const int bs = block_size(type_id);
    if (cols % bs != 0)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len,
                    "Element count %lld is not a multiple of block size %d for type %s",
                    (long long)cols, bs, type_label(type_id));
    const int64_t expect = cols / bs * block_bytes(type_id);
    if (row_bytes != expect)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len,
                    "Row byte size %lld does not match %lld for %lld %s columns",
                    (long long)row_bytes, (long long)expect, (long long)cols,
                    type_label(type_id));
    return GOLLEK_HIP_OK;
}

// Host buffers (a Java float[], a numpy array) are pageable; copies through
// page-locked staging run as plain DMA.  Up to kHostStageMax bytes per
// handle (grown on demand, freed with the handle); larger transfers copy
// from the caller's memory directly.  Every host entry point synchronizes
// its stream before returning, so a buffer is never regrown under a copy.
constexpr size_t kHostStageMax = (size_t)16 << 20;

uint8_t *host_staging(gollek_hip_weight *w, size_t bytes) {
    if (bytes > kHostStageMax) return nullptr;
    if (w->hstage_bytes >= bytes) return w->hstage;
    if (w->hstage != nullptr) (void)hipHostFree(w->hstage);
    w->hstage = nullptr;
    w->hstage_bytes = 0;
    const size_t want = bytes < ((size_t)64 << 10) ? ((size_t)64 << 10) : bytes;
    void *p = nullptr;
    if (hipHostMalloc(&p, want, hipHostMallocDefault) != hipSuccess) {
        (void)hipGetLastError();
        return nullptr;  // the direct copies still work
    }
    w->hstage = static_cast<uint8_t *>(p);
    w->hstage_bytes = want;
    return w->hstage;
}

// Copies 16-byte units [0, na) and [na + gap, na + gap + nb) from the pinned
// staging (mapped for the device) to the same offsets of device memory: for
// the kilobytes of a call's inputs one kernel launch starts sooner than a
// DMA-engine copy, and the gap (an output region) does not cross the bus.
__global__ __launch_bounds__(256) void pull_staging_kernel(const uint4 *__restrict__ src, uint4 *__restrict__ dst,
                                                           int64_t na, int64_t gap, int64_t nb) {
    int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= na + nb) return;
    if (i >= na) i += gap;
    dst[i] = src[i];
}

// dst <- bytes [0, a) and [a + gap, a + gap + b) of the pinned staging at
// src (offsets and pointers 16-byte aligned for the kernel): the pull kernel
// up to kPullMax bytes, the DMA engine otherwise.
constexpr size_t kPullMax = (size_t)1 << 20;
hipError_t pull_staging(void *dst, const void *src, size_t a, hipStream_t stream, size_t gap = 0, size_t b = 0) {
    if (a + b == 0) return hipSuccess;
    const bool kernel = a + b <= kPullMax && (a | gap | b) % 16 == 0 &&
                        ((reinterpret_cast<uintptr_t>(dst) | reinterpret_cast<uintptr_t>(src)) & 15u) == 0;
    if (!kernel) {
        hipError_t e = hipMemcpyAsync(dst, src, a, hipMemcpyHostToDevice, stream);
        if (e == hipSuccess && b > 0)
            e = hipMemcpyAsync(static_cast<uint8_t *>(dst) + a + gap, static_cast<const uint8_t *>(src) + a + gap, b,
                               hipMemcpyHostToDevice, stream);
        return e;
    }
    const int64_t n = (int64_t)((a + b) / 16);
    hipLaunchKernelGGL(pull_staging_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream,
                       reinterpret_cast<const uint4 *>(src), reinterpret_cast<uint4 *>(dst), (int64_t)(a / 16),
                       (int64_t)(gap / 16), (int64_t)(b / 16));
    return hipGetLastError();
}

int32_t ensure_staging(gollek_hip_weight *w, size_t bytes, char *err, size_t err_len) {
    if (w->staging_bytes >= bytes) return GOLLEK_HIP_OK;
    if (w->staging != nullptr) {
        (void)hipFree(w->staging);
        w->staging = nullptr;
        w->staging_bytes = 0;
    }
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&w->staging), bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(staging)", err, err_len);
    w->staging_bytes = bytes;
    return GOLLEK_HIP_OK;
}

size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// A compact handle's device temporaries (grown on demand; the _device entries
// that use them must not overlap on one handle).
int32_t ensure_ctmp(gollek_hip_weight *w, size_t bytes, char *err, size_t err_len) {
    if (w->ctmp_bytes >= bytes) return GOLLEK_HIP_OK;
    if (w->ctmp != nullptr) {
        (void)hipFree(w->ctmp);
        w->ctmp = nullptr;
        w->ctmp_bytes = 0;
    }
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&w->ctmp), bytes);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(compact temporaries)", err, err_len);
    w->ctmp_bytes = bytes;
    return GOLLEK_HIP_OK;
}

int32_t compact_unsupported(const gollek_hip_weight *w, const char *what, char *err, size_t err_len) {
    return fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len,
                "%s reads GGUF rows, which a compacted handle (type %d, %lld x %lld) no longer holds", what,
                w->type_id, (long long)w->rows, (long long)w->cols);
}

gollek_hip_weight *make_weight(int32_t type_id, int64_t rows, int64_t cols, int64_t row_bytes,
                               char *err, size_t err_len) {
    if (check_shape(type_id, rows, cols, row_bytes, err, err_len) != GOLLEK_HIP_OK) return nullptr;
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) {
        hip_fail(e, "hipGetDevice", err, err_len);
        return nullptr;
    }
    if (use_device(device, err, err_len) != GOLLEK_HIP_OK) return nullptr;
    gollek_hip_weight *w = new (std::nothrow) gollek_hip_weight();
    if (w == nullptr) {
        fail(GOLLEK_HIP_ERR_NOMEM, err, err_len, "out of host memory");
        return nullptr;
    }
    w->type_id = type_id;
    w->rows = rows;
    w->cols = cols;
    w->row_bytes = row_bytes;
    w->device = device;
    e = hipStreamCreateWithFlags(&w->stream, hipStreamNonBlocking);
    if (e != hipSuccess) {
        hip_fail(e, "hipStreamCreate", err, err_len);
        delete w;
        return nullptr;
    }
    return w;
}

}  // namespace

extern "C" {

int32_t gollek_hip_version(void) { return kAbiVersion; }

int32_t gollek_hip_init(int32_t device, char *err, size_t err_len) {
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess) return hip_fail(e, "hipGetDeviceCount", err, err_len);
    if (device < 0 || device >= count)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Device %d is outside [0, %d)", device, count);
    const int32_t rc = use_device(device, err, err_len);
    if (rc == GOLLEK_HIP_OK) ok(err, err_len);
    return rc;
}

const char *gollek_hip_last_error(void) { return g_last_error.c_str(); }

int32_t gollek_hip_last_status(void) { return g_last_status; }

int32_t gollek_hip_testing_set_option(const char *key, int64_t value, char *err, size_t err_len) {
    if (key == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "key");
    gollek::LaunchTuning &t = gollek::tuning();
    if (strcmp(key, "gemv_variant") == 0 && (value == 0 || value == 1 || value == 3 || value == 4))
        t.gemv_variant = (int)value;
    else if (strcmp(key, "moe_variant") == 0 && (value == 0 || value == 1)) t.moe_variant = (int)value;
    else return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Unknown option %s = %lld", key, (long long)value);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

gollek_hip_weight *gollek_hip_weight_upload(int32_t type_id, const void *host_bytes, int64_t rows,
                                            int64_t cols, int64_t row_bytes, char *err,
                                            size_t err_len) {
    if (host_bytes == nullptr) {
        fail(GOLLEK_HIP_ERR_NULL, err, err_len, "host_bytes");
        return nullptr;
    }
    gollek_hip_weight *w = make_weight(type_id, rows, cols, row_bytes, err, err_len);
    if (w == nullptr) return nullptr;
    const size_t bytes = (size_t)rows * (size_t)row_bytes;
    if (bytes > 0) {
        hipError_t e = hipMalloc(reinterpret_cast<void **>(&w->data), bytes);
        if (e == hipSuccess) e = hipMemcpy(w->data, host_bytes, bytes, hipMemcpyHostToDevice);
        if (e != hipSuccess) {
            hip_fail(e, "weight upload", err, err_len);
            gollek_hip_weight_free(w);
            return nullptr;
        }
    }
    w->owned = true;
    ok(err, err_len);
    return w;
}

gollek_hip_weight *gollek_hip_weight_wrap_device(int32_t type_id, const void *device_bytes,
                                                 int64_t rows, int64_t cols, int64_t row_bytes,
                                                 char *err, size_t err_len) {
    if (device_bytes == nullptr) {
        fail(GOLLEK_HIP_ERR_NULL, err, err_len, "device_bytes");
        return nullptr;
    }
    gollek_hip_weight *w = make_weight(type_id, rows, cols, row_bytes, err, err_len);
    if (w == nullptr) return nullptr;
    w->data = const_cast<uint8_t *>(static_cast<const uint8_t *>(device_bytes));
    w->owned = false;
    ok(err, err_len);
    return w;
}

void gollek_hip_weight_free(gollek_hip_weight *w) {
    if (w == nullptr) return;
    (void)hipSetDevice(w->device);
    if (w->stream != nullptr) (void)hipStreamSynchronize(w->stream);
    if (w->owned && w->data != nullptr) (void)hipFree(w->data);
    if (w->staging != nullptr) (void)hipFree(w->staging);
    if (w->gemm_ws != nullptr) (void)hipFree(w->gemm_ws);
    if (w->prep != nullptr) (void)hipFree(w->prep);
    if (w->ctmp != nullptr) (void)hipFree(w->ctmp);
    if (w->hstage != nullptr) (void)hipHostFree(w->hstage);
    if (w->stream != nullptr) (void)hipStreamDestroy(w->stream);
    delete w;
}

int32_t gollek_hip_weight_prepare(gollek_hip_weight *w, char *err, size_t err_len) {
    if (w == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "tensor");
    std::lock_guard<std::mutex> lock(w->mu);
    int32_t rc = use_device(w->device, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    // Only shapes the column kernel takes for a full mat-vec have a layout.
    const int64_t per = gollek::col_layout_rows(w->type_id, w->rows, w->cols);
    if (w->compact) {  // its layout is all it holds
        if (per == w->prep_rows) {
            ok(err, err_len);
            return GOLLEK_HIP_OK;
        }
        return fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len,
                    "compacted handle: its prepared layout is for %lld rows per workgroup, the kernels now use %lld",
                    (long long)w->prep_rows, (long long)per);
    }
    const bool takes = per > 0 && (gollek::q32_mfma_supported(w->type_id, w->row_bytes, w->cols, w->rows, w->data,
                                                              nullptr) ||
                                   (w->type_id == GOLLEK_HIP_Q4_K &&
                                    gollek::q4k_mfma_supported(w->row_bytes, w->cols, w->rows, w->data, nullptr)));
    if (!takes || (w->prep != nullptr && w->prep_rows == per)) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    if (w->prep != nullptr) {
        (void)hipStreamSynchronize(w->stream);
        (void)hipFree(w->prep);
        w->prep = nullptr;
        w->prep_rows = 0;
    }
    uint8_t *p = nullptr;
    hipError_t e = hipMalloc(reinterpret_cast<void **>(&p), (size_t)(w->rows * w->row_bytes));
    if (e != hipSuccess) {
        (void)hipGetLastError();
        return fail(GOLLEK_HIP_ERR_NOMEM, err, err_len, "prepared layout of %lld bytes",
                    (long long)(w->rows * w->row_bytes));
    }
    e = gollek::launch_prepare_col_layout(w->type_id, w->data, p, w->rows, w->row_bytes, per, w->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
    if (e != hipSuccess) {
        (void)hipFree(p);
        return hip_fail(e, "prepare", err, err_len);
    }
    w->prep = p;
    w->prep_rows = per;
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_weight_unprepare(gollek_hip_weight *w, char *err, size_t err_len) {
    if (w == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "tensor");
    std::lock_guard<std::mutex> lock(w->mu);
    if (w->compact) {
        // The GGUF rows are rebuilt from the layout first.
        const int32_t rc = use_device(w->device, err, err_len);
        if (rc != GOLLEK_HIP_OK) return rc;
        uint8_t *d = nullptr;
        const size_t bytes = (size_t)(w->rows * w->row_bytes);
        hipError_t e = hipMalloc(reinterpret_cast<void **>(&d), bytes);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(GGUF rows)", err, err_len);
        e = gollek::launch_gather_col_rows(w->type_id, w->prep, d, w->rows, w->row_bytes, w->prep_rows, 0, w->rows,
                                           w->stream);
        if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
        if (e != hipSuccess) {
            (void)hipFree(d);
            return hip_fail(e, "unprepare (rebuild GGUF rows)", err, err_len);
        }
        w->data = d;
        w->compact = false;
    }
    if (w->prep != nullptr) {
        const int32_t rc = use_device(w->device, err, err_len);
        if (rc != GOLLEK_HIP_OK) return rc;
        // The host entries' launches that read the copy ran on this stream.
        hipError_t e = hipStreamSynchronize(w->stream);
        if (e == hipSuccess) e = hipFree(w->prep);
        w->prep = nullptr;
        w->prep_rows = 0;
        if (e != hipSuccess) return hip_fail(e, "unprepare", err, err_len);
    }
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_weight_compact(gollek_hip_weight *w, char *err, size_t err_len) {
    if (w == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "tensor");
    std::lock_guard<std::mutex> lock(w->mu);
    if (w->compact) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    if (!w->owned)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "the handle borrows its bytes (wrap_device): nothing to free");
    if (w->prep == nullptr)
        return fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len,
                    "no prepared layout to keep (prepare first; type %d, %lld x %lld has none when prepare is a no-op)",
                    w->type_id, (long long)w->rows, (long long)w->cols);
    const int32_t rc = use_device(w->device, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    hipError_t e = hipStreamSynchronize(w->stream);
    if (e == hipSuccess && w->data != nullptr) e = hipFree(w->data);
    if (e != hipSuccess) return hip_fail(e, "compact", err, err_len);
    w->data = nullptr;
    w->compact = true;
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_weight_info(const gollek_hip_weight *w, int32_t *type_id, int64_t *rows,
                               int64_t *cols, int64_t *row_bytes) {
    if (w == nullptr) return GOLLEK_HIP_ERR_NULL;
    if (type_id) *type_id = w->type_id;
    if (rows) *rows = w->rows;
    if (cols) *cols = w->cols;
    if (row_bytes) *row_bytes = w->row_bytes;
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_dequantize_rows(gollek_hip_weight *w, int64_t row0, int64_t nrows, float *dst,
                                   int64_t dst_len, char *err, size_t err_len) {
    if (w == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "tensor");
    if (dst == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "dst");
    if (nrows < 0) return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Row count %lld is negative", (long long)nrows);
    if (dst_len < nrows * w->cols)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Vector length %lld is smaller than columns %lld",
                    (long long)dst_len, (long long)(nrows * w->cols));
    if (row0 < 0 || row0 + nrows > w->rows || (nrows > 0 && row0 >= w->rows))
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Row %lld is outside tensor row count %lld",
                    (long long)(row0 < 0 || row0 >= w->rows ? row0 : row0 + nrows - 1),
                    (long long)w->rows);
    if (nrows == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    std::lock_guard<std::mutex> lock(w->mu);
    int32_t rc = use_device(w->device, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    const size_t bytes = (size_t)nrows * (size_t)w->cols * sizeof(float);
    // A compact handle's rows are first gathered from its prepared layout
    // into device staging (the same bytes, so the same bits).
    const size_t gbytes = w->compact ? align_up((size_t)(nrows * w->row_bytes), 256) : 0;
    // With the pinned staging the kernel stores the rows there itself (the
    // buffer is mapped for the device); otherwise through device staging and
    // a device-to-host copy.
    uint8_t *hs = host_staging(w, bytes);
    float *d_out = reinterpret_cast<float *>(hs);
    if (hs == nullptr || gbytes > 0) {
        rc = ensure_staging(w, gbytes + (hs == nullptr ? bytes : 0), err, err_len);
        if (rc != GOLLEK_HIP_OK) return rc;
        if (hs == nullptr) d_out = reinterpret_cast<float *>(w->staging + gbytes);
    }
    const uint8_t *src = w->data;
    int64_t srow0 = row0;
    hipError_t e = hipSuccess;
    if (w->compact) {
        e = gollek::launch_gather_col_rows(w->type_id, w->prep, w->staging, w->rows, w->row_bytes, w->prep_rows,
                                           row0, nrows, w->stream);
        src = w->staging;
        srow0 = 0;
    }
    if (e == hipSuccess)
        e = gollek::launch_dequant(w->type_id, src, w->row_bytes, w->cols, srow0, nrows, d_out, w->stream);
    if (e == hipSuccess && hs == nullptr)
        e = hipMemcpyAsync(dst, d_out, bytes, hipMemcpyDeviceToHost, w->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
    if (e != hipSuccess) return hip_fail(e, "dequantize", err, err_len);
    if (hs != nullptr) std::memcpy(dst, hs, bytes);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

// Rows row0 .. row0 + nrows - 1 of W x.  A compact handle runs the full
// mat-vec from its prepared layout and returns the requested rows (the same
// bits as its full call).
static int32_t matvec_host(gollek_hip_weight *w, int64_t row0, int64_t nrows, const float *x, float *y,
                           char *err, size_t err_len) {
    std::lock_guard<std::mutex> lock(w->mu);
    int32_t rc = use_device(w->device, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    const int64_t krows = w->compact ? w->rows : nrows;  // rows the kernel computes
    const size_t x_bytes = align_up((size_t)w->cols * sizeof(float), 256);
    const size_t y_bytes = (size_t)krows * sizeof(float);
    rc = ensure_staging(w, x_bytes + y_bytes, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    float *d_x = reinterpret_cast<float *>(w->staging);
    float *d_y = reinterpret_cast<float *>(w->staging + x_bytes);
    const size_t xn = (size_t)w->cols * sizeof(float);
    uint8_t *hs = host_staging(w, x_bytes + y_bytes);
    if (hs != nullptr) std::memcpy(hs, x, xn);
    hipError_t e = hs != nullptr ? pull_staging(d_x, hs, xn, w->stream)
                                 : hipMemcpyAsync(d_x, x, xn, hipMemcpyHostToDevice, w->stream);
    // the prepared layout covers full mat-vecs only (its partition depends on the row count)
    const bool full = row0 == 0 && nrows == w->rows;
    // With the pinned staging the kernel stores y there itself (the buffer is
    // mapped for the device; the stream synchronisation below makes the
    // stores visible to the host), which saves the device-to-host copy.
    float *k_y = hs != nullptr ? reinterpret_cast<float *>(hs + x_bytes) : d_y;
    if (e == hipSuccess && w->compact) {
        e = gollek::launch_gemv_prepared(w->type_id, w->prep, w->row_bytes, w->cols, d_x, k_y, w->rows, w->prep_rows,
                                         w->stream);
        if (e == hipErrorInvalidValue)
            return fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len,
                        "compacted handle: the column kernel's partition is no longer its layout's");
    } else if (e == hipSuccess) {
        e = gollek::launch_gemv(w->type_id, w->data + row0 * w->row_bytes, w->row_bytes, w->cols, d_x, k_y, nrows,
                                w->stream, full ? w->prep : nullptr, full ? w->prep_rows : 0);
    }
    const int64_t first = w->compact ? row0 : 0;  // the caller's rows in the kernel's y
    const size_t out_bytes = (size_t)nrows * sizeof(float);
    if (e == hipSuccess && hs == nullptr)
        e = hipMemcpyAsync(y, d_y + first, out_bytes, hipMemcpyDeviceToHost, w->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
    if (e != hipSuccess) return hip_fail(e, "matvec", err, err_len);
    if (hs != nullptr) std::memcpy(y, hs + x_bytes + first * sizeof(float), out_bytes);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_dot_row(gollek_hip_weight *w, int64_t row, const float *x, int64_t x_len,
                           float *out, char *err, size_t err_len) {
    if (w == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "tensor");
    if (x == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "vector");
    if (out == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "output");
    if (x_len < w->cols)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Vector length %lld is smaller than columns %lld",
                    (long long)x_len, (long long)w->cols);
    if (row < 0 || row >= w->rows)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Row %lld is outside tensor row count %lld",
                    (long long)row, (long long)w->rows);
    return matvec_host(w, row, 1, x, out, err, err_len);
}

int32_t gollek_hip_matvec_rows(gollek_hip_weight *w, const float *x, int64_t x_len, float *y,
                               int64_t y_len, int64_t row_count, char *err, size_t err_len) {
    // RT/GgufMatVec.java:40-75: null checks, vector length, row count,
    // output length, then the row_count == 0 no-op.
    if (w == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "tensor");
    if (x == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "vector");
    if (y == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "output");
    if (x_len < w->cols)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Vector length %lld is smaller than columns %lld",
                    (long long)x_len, (long long)w->cols);
    if (row_count < 0 || row_count > w->rows)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Requested row count %lld is outside tensor rows %lld",
                    (long long)row_count, (long long)w->rows);
    if (y_len < row_count)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Output length %lld is smaller than requested rows %lld",
                    (long long)y_len, (long long)row_count);
    if (row_count == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    return matvec_host(w, 0, row_count, x, y, err, err_len);
}

int32_t gollek_hip_dequantize_rows_device(gollek_hip_weight *w, int64_t row0, int64_t nrows,
                                          float *dst, void *stream, char *err, size_t err_len) {
    if (w == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "tensor");
    if (dst == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "dst");
    if (nrows < 0 || row0 < 0 || row0 + nrows > w->rows)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Rows [%lld, %lld) are outside tensor row count %lld",
                    (long long)row0, (long long)(row0 + nrows), (long long)w->rows);
    const hipStream_t st = static_cast<hipStream_t>(stream);
    const uint8_t *src = w->data;
    int64_t srow0 = row0;
    hipError_t e = hipSuccess;
    if (w->compact && nrows > 0) {  // the rows gathered from the prepared layout first
        {
            std::lock_guard<std::mutex> lock(w->mu);
            const int32_t rc = ensure_ctmp(w, (size_t)(nrows * w->row_bytes), err, err_len);
            if (rc != GOLLEK_HIP_OK) return rc;
        }
        e = gollek::launch_gather_col_rows(w->type_id, w->prep, w->ctmp, w->rows, w->row_bytes, w->prep_rows, row0,
                                           nrows, st);
        src = w->ctmp;
        srow0 = 0;
    }
    if (e == hipSuccess) e = gollek::launch_dequant(w->type_id, src, w->row_bytes, w->cols, srow0, nrows, dst, st);
    if (e != hipSuccess) return hip_fail(e, "dequantize launch", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_matvec_device(gollek_hip_weight *w, const float *x, float *y,
                                 int64_t row_count, void *stream, char *err, size_t err_len) {
    if (w == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "tensor");
    if (x == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "vector");
    if (y == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "output");
    if (row_count < 0 || row_count > w->rows)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Requested row count %lld is outside tensor rows %lld",
                    (long long)row_count, (long long)w->rows);
    const bool full = row_count == w->rows;  // the prepared layout covers full mat-vecs only
    const hipStream_t st = static_cast<hipStream_t>(stream);
    hipError_t e = hipSuccess;
    if (w->compact && row_count > 0) {
        // The full mat-vec from the prepared layout; a prefix goes through a
        // temporary y, an unaligned x through an aligned copy.
        const bool x_ok = (reinterpret_cast<uintptr_t>(x) & 15u) == 0;
        const size_t x_bytes = x_ok ? 0 : align_up((size_t)w->cols * sizeof(float), 256);
        const size_t need = x_bytes + (full ? 0 : (size_t)w->rows * sizeof(float));
        if (need > 0) {
            std::lock_guard<std::mutex> lock(w->mu);
            const int32_t rc = ensure_ctmp(w, need, err, err_len);
            if (rc != GOLLEK_HIP_OK) return rc;
        }
        const float *kx = x;
        if (!x_ok) {
            e = hipMemcpyAsync(w->ctmp, x, (size_t)w->cols * sizeof(float), hipMemcpyDeviceToDevice, st);
            kx = reinterpret_cast<const float *>(w->ctmp);
        }
        float *ky = full ? y : reinterpret_cast<float *>(w->ctmp + x_bytes);
        if (e == hipSuccess)
            e = gollek::launch_gemv_prepared(w->type_id, w->prep, w->row_bytes, w->cols, kx, ky, w->rows,
                                             w->prep_rows, st);
        if (e == hipErrorInvalidValue)
            return fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len,
                        "compacted handle: the column kernel's partition is no longer its layout's");
        if (e == hipSuccess && !full)
            e = hipMemcpyAsync(y, ky, (size_t)row_count * sizeof(float), hipMemcpyDeviceToDevice, st);
    } else if (!w->compact) {
        e = gollek::launch_gemv(w->type_id, w->data, w->row_bytes, w->cols, x, y, row_count, st,
                                full ? w->prep : nullptr, full ? w->prep_rows : 0);
    }
    if (e != hipSuccess) return hip_fail(e, "matvec launch", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

// x_dev: whether the kernels read x where the caller put it (the _device
// entries) rather than from the staging buffer.
static int32_t check_gemm(gollek_hip_weight *w, const void *x, const void *y, int64_t m, bool x_dev,
                          char *err, size_t err_len) {
    if (w == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "tensor");
    if (x == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "input");
    if (y == nullptr) return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "output");
    if (w->type_id != GOLLEK_HIP_Q8_0 && w->type_id != GOLLEK_HIP_Q4_0 && w->type_id != GOLLEK_HIP_Q4_K &&
        w->type_id != GOLLEK_HIP_Q5_K && w->type_id != GOLLEK_HIP_Q6_K)
        return fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len,
                    "Unsupported GGUF bf16 GEMM type id: %d (Q8_0, Q4_0, Q4_K, Q5_K or Q6_K)", w->type_id);
    // A compacted handle holds the prepared column layout only, which the
    // GEMM reads for up to four rows of X while its partition is still the
    // column kernel's.
    if (w->compact && !(m >= 0 && m <= 4 && w->rows <= 0x7FFFFFFF && w->cols <= 0x7FFFFFFF &&
                        gollek::col_layout_rows(w->type_id, w->rows, w->cols) == w->prep_rows &&
                        (m == 0 || gollek::gemm_col_supported(w->type_id, w->row_bytes, (int)m, (int)w->rows,
                                                              (int)w->cols, w->prep, x_dev ? x : w->prep))))
        return compact_unsupported(w, "GEMM past 4 rows of X (or of 8-byte misaligned X)", err, err_len);
    if (m < 0 || m > (int64_t)0x7FFFFFFF || w->rows > 0x7FFFFFFF || w->cols > 0x7FFFFFFF)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "GEMM shape %lld x %lld x %lld is out of range",
                    (long long)m, (long long)w->rows, (long long)w->cols);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_gemm_bf16(gollek_hip_weight *w, const uint16_t *x, int64_t x_len, int64_t m,
                             float *y, int64_t y_len, char *err, size_t err_len) {
    int32_t rc = check_gemm(w, x, y, m, false, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    if (x_len < m * w->cols)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Input length %lld is smaller than %lld x %lld",
                    (long long)x_len, (long long)m, (long long)w->cols);
    if (y_len < m * w->rows)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Output length %lld is smaller than %lld x %lld",
                    (long long)y_len, (long long)m, (long long)w->rows);
    if (m == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    std::lock_guard<std::mutex> lock(w->mu);
    rc = use_device(w->device, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    const size_t x_bytes = align_up((size_t)(m * w->cols) * sizeof(uint16_t), 256);
    const size_t y_bytes = (size_t)(m * w->rows) * sizeof(float);
    const size_t ws_bytes = gollek::gemm_workspace_bytes(w->type_id, (int)m, (int)w->rows, (int)w->cols);
    const size_t ws_off = align_up(x_bytes + y_bytes, 256);
    rc = ensure_staging(w, ws_off + ws_bytes, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    uint16_t *d_x = reinterpret_cast<uint16_t *>(w->staging);
    float *d_y = reinterpret_cast<float *>(w->staging + x_bytes);
    float *d_ws = ws_bytes ? reinterpret_cast<float *>(w->staging + ws_off) : nullptr;
    const size_t xn = (size_t)(m * w->cols) * sizeof(uint16_t);
    uint8_t *hs = host_staging(w, x_bytes + y_bytes);
    if (hs != nullptr) std::memcpy(hs, x, xn);
    hipError_t e = hs != nullptr ? pull_staging(d_x, hs, xn, w->stream)
                                 : hipMemcpyAsync(d_x, x, xn, hipMemcpyHostToDevice, w->stream);
    // With the pinned staging the kernels store Y there themselves (mapped
    // for the device; x_bytes keeps it 256-byte aligned, so the split-K
    // path stays available), which saves the device-to-host copy.
    float *k_y = hs != nullptr ? reinterpret_cast<float *>(hs + x_bytes) : d_y;
    if (e == hipSuccess)
        e = gollek::launch_gemm_bf16(w->type_id, w->data, w->row_bytes, d_x, k_y, (int)m, (int)w->rows,
                                     (int)w->cols, w->stream, d_ws, ws_bytes, w->prep, w->prep_rows);
    if (e == hipSuccess && hs == nullptr)
        e = hipMemcpyAsync(y, d_y, y_bytes, hipMemcpyDeviceToHost, w->stream);
    if (e == hipSuccess) e = hipStreamSynchronize(w->stream);
    if (e != hipSuccess) return hip_fail(e, "gemm", err, err_len);
    if (hs != nullptr) std::memcpy(y, hs + x_bytes, y_bytes);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_gemm_bf16_device(gollek_hip_weight *w, const uint16_t *x, int64_t m, float *y,
                                    void *stream, char *err, size_t err_len) {
    const int32_t rc = check_gemm(w, x, y, m, true, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    // The handle's split-K workspace: allocated at the first call that splits,
    // for the largest split any m of this weight uses (below 16 MiB on 256
    // CUs), and kept until the handle is freed, so a launch in flight never
    // loses it.
    const size_t need = gollek::gemm_workspace_bytes(w->type_id, (int)m, (int)w->rows, (int)w->cols);
    if (need > 0) {
        std::lock_guard<std::mutex> lock(w->mu);
        if (w->gemm_ws == nullptr) {
            const size_t most = gollek::gemm_workspace_max_bytes(w->type_id, (int)w->rows, (int)w->cols);
            const size_t bytes = most > need ? most : need;
            const int32_t urc = use_device(w->device, err, err_len);
            if (urc != GOLLEK_HIP_OK) return urc;
            const hipError_t ae = hipMalloc(reinterpret_cast<void **>(&w->gemm_ws), bytes);
            if (ae != hipSuccess) {
                w->gemm_ws = nullptr;
                return hip_fail(ae, "hipMalloc(gemm workspace)", err, err_len);
            }
            w->gemm_ws_bytes = bytes;
        }
    }
    hipError_t e = gollek::launch_gemm_bf16(w->type_id, w->data, w->row_bytes, x, y, (int)m, (int)w->rows,
                                            (int)w->cols, static_cast<hipStream_t>(stream),
                                            need ? w->gemm_ws : nullptr, w->gemm_ws_bytes, w->prep, w->prep_rows);
    if (e != hipSuccess) return hip_fail(e, "gemm launch", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_gemm_bf16_device_noalloc(gollek_hip_weight *w, const uint16_t *x, int64_t m,
                                            float *y, void *stream, char *err, size_t err_len) {
    const int32_t rc = check_gemm(w, x, y, m, true, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    // The split-K partials go to this GPU's static scratch: no allocation,
    // and every call on the GPU shares it (each split writes its whole
    // partial tile before the in-order reduction reads it, so nothing needs
    // clearing; overlapping calls race).  A shape whose splits would need more
    // than the scratch holds is split less (the launcher picks the splits
    // that fit), down to none.
    const size_t need = gollek::gemm_workspace_bytes(w->type_id, (int)m, (int)w->rows, (int)w->cols);
    float *ws = nullptr;
    if (need > 0) {
        ws = (w->device >= 0 && w->device < kMaxDevices) ? g_scratch_ptr[w->device].load() : nullptr;
        if (ws == nullptr)
            return fail(GOLLEK_HIP_ERR_DEVICE, err, err_len,
                        "the static GEMM scratch of device %d is not set up", w->device);
    }
    hipError_t e = gollek::launch_gemm_bf16(w->type_id, w->data, w->row_bytes, x, y, (int)m, (int)w->rows,
                                            (int)w->cols, static_cast<hipStream_t>(stream), ws,
                                            ws != nullptr ? kGemmScratchBytes : 0, w->prep, w->prep_rows);
    if (e != hipSuccess) return hip_fail(e, "gemm launch", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

struct MoeShape {
    int E, H, I;
    int down_type;
};

static bool moe_type(int32_t t) {
    return t == GOLLEK_HIP_Q4_0 || t == GOLLEK_HIP_Q8_0 || t == GOLLEK_HIP_Q4_K || t == GOLLEK_HIP_Q5_K ||
           t == GOLLEK_HIP_Q6_K;
}

// The grouped expert FFN on the kernels that take the types and shape.
static hipError_t moe_launch(const MoeShape &sh, gollek_hip_weight *gate, gollek_hip_weight *up,
                             gollek_hip_weight *down, const float *x, const int32_t *ids, const float *w,
                             int64_t tokens, int64_t top_k, float *out, uint8_t *ws, hipStream_t s) {
    return gollek::launch_moe(gate->type_id, up->type_id, down->type_id, gate->data, up->data, down->data,
                              gate->row_bytes, up->row_bytes, down->row_bytes, sh.E, sh.H, sh.I, x, ids, w,
                              (int)tokens, (int)top_k, out, ws, s);
}

static int32_t check_moe(gollek_hip_weight *gate, gollek_hip_weight *up, gollek_hip_weight *down,
                         int64_t n_experts, int64_t tokens, int64_t top_k, MoeShape *shape,
                         char *err, size_t err_len) {
    if (gate == nullptr || up == nullptr || down == nullptr)
        return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "expert weights");
    for (const gollek_hip_weight *t : {gate, up, down})
        if (t->compact) return compact_unsupported(t, "The MoE expert FFN", err, err_len);
    if (!moe_type(gate->type_id) || !moe_type(up->type_id) || !moe_type(down->type_id))
        return fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len,
                    "Unsupported MoE expert weight types %d/%d/%d (Q8_0, Q4_0, Q4_K, Q5_K or Q6_K)",
                    gate->type_id, up->type_id, down->type_id);
    if (n_experts <= 0 || gate->rows % n_experts != 0)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Gate rows %lld are not a multiple of %lld experts",
                    (long long)gate->rows, (long long)n_experts);
    const int64_t H = gate->cols, I = gate->rows / n_experts;
    if (up->rows != gate->rows || up->cols != H || down->rows != n_experts * H || down->cols != I)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len,
                    "Expert shapes disagree: gate %lldx%lld up %lldx%lld down %lldx%lld",
                    (long long)gate->rows, (long long)gate->cols, (long long)up->rows,
                    (long long)up->cols, (long long)down->rows, (long long)down->cols);
    if (tokens < 0 || top_k <= 0 || tokens * top_k > (1 << 24))
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Invalid tokens %lld / top_k %lld",
                    (long long)tokens, (long long)top_k);
    shape->E = (int)n_experts;
    shape->H = (int)H;
    shape->I = (int)I;
    shape->down_type = down->type_id;
    return GOLLEK_HIP_OK;
}

int64_t gollek_hip_moe_workspace_bytes(int64_t tokens, int64_t top_k, int64_t hidden,
                                       int64_t inter, int64_t n_experts) {
    if (tokens < 0 || top_k <= 0 || hidden <= 0 || inter <= 0 || n_experts <= 0) return -1;
    return (int64_t)gollek::moe_layout(tokens, top_k, hidden, inter, n_experts).total;
}

int32_t gollek_hip_moe_grouped_device(gollek_hip_weight *gate, gollek_hip_weight *up,
                                      gollek_hip_weight *down, int64_t n_experts, const float *x,
                                      const int32_t *ids, const float *weights, int64_t tokens,
                                      int64_t top_k, float *out, void *workspace,
                                      int64_t workspace_bytes, void *stream, char *err,
                                      size_t err_len) {
    MoeShape sh;
    int32_t rc = check_moe(gate, up, down, n_experts, tokens, top_k, &sh, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    if (tokens == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    if (x == nullptr || ids == nullptr || weights == nullptr || out == nullptr || workspace == nullptr)
        return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "MoE buffers");
    const int64_t need = gollek_hip_moe_workspace_bytes(tokens, top_k, sh.H, sh.I, sh.E);
    if (workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len,
                    "Workspace of %lld bytes (256-byte aligned) needed, got %lld",
                    (long long)need, (long long)workspace_bytes);
    hipError_t e = moe_launch(sh, gate, up, down, x, ids, weights, tokens, top_k, out,
                              static_cast<uint8_t *>(workspace), static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "moe launch", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_moe_grouped(gollek_hip_weight *gate, gollek_hip_weight *up,
                               gollek_hip_weight *down, int64_t n_experts, const float *x,
                               int64_t tokens, const int32_t *ids, const float *weights,
                               int64_t top_k, float *out, int64_t out_len, char *err,
                               size_t err_len) {
    MoeShape sh;
    int32_t rc = check_moe(gate, up, down, n_experts, tokens, top_k, &sh, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    if (x == nullptr || ids == nullptr || weights == nullptr || out == nullptr)
        return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "MoE buffers");
    if (out_len < tokens * sh.H)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Output length %lld is smaller than %lld x %d",
                    (long long)out_len, (long long)tokens, sh.H);
    if (tokens == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    std::lock_guard<std::mutex> lock(gate->mu);
    rc = use_device(gate->device, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    const size_t xb = align_up((size_t)(tokens * sh.H) * 4, 256);
    const size_t rb = align_up((size_t)(tokens * top_k) * 4, 256);
    const size_t ws = (size_t)gollek_hip_moe_workspace_bytes(tokens, top_k, sh.H, sh.I, sh.E);
    rc = ensure_staging(gate, 2 * xb + 2 * rb + ws, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    uint8_t *base = gate->staging;
    float *d_x = reinterpret_cast<float *>(base);
    float *d_out = reinterpret_cast<float *>(base + xb);
    int32_t *d_ids = reinterpret_cast<int32_t *>(base + 2 * xb);
    float *d_w = reinterpret_cast<float *>(base + 2 * xb + rb);
    uint8_t *d_ws = base + 2 * xb + 2 * rb;
    hipStream_t s = gate->stream;
    const size_t xn = (size_t)(tokens * sh.H) * 4, rn = (size_t)(tokens * top_k) * 4;
    // Pinned staging laid out as the device buffer (x | out | ids | weights):
    // the inputs go up in one copy and the kernels store `out` into it.
    uint8_t *hs = host_staging(gate, 2 * xb + 2 * rb);
    hipError_t e = hipSuccess;
    if (hs != nullptr) {
        std::memcpy(hs, x, xn);
        std::memcpy(hs + 2 * xb, ids, rn);
        std::memcpy(hs + 2 * xb + rb, weights, rn);
        e = pull_staging(d_x, hs, xn, s, 2 * xb - xn, 2 * rb);
    } else {
        e = hipMemcpyAsync(d_x, x, xn, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipMemcpyAsync(d_ids, ids, rn, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipMemcpyAsync(d_w, weights, rn, hipMemcpyHostToDevice, s);
    }
    float *k_out = hs != nullptr ? reinterpret_cast<float *>(hs + xb) : d_out;
    if (e == hipSuccess)
        e = moe_launch(sh, gate, up, down, d_x, d_ids, d_w, tokens, top_k, k_out, d_ws, s);
    if (e == hipSuccess && hs == nullptr) e = hipMemcpyAsync(out, d_out, xn, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "moe", err, err_len);
    if (hs != nullptr) std::memcpy(out, hs + xb, xn);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int64_t gollek_hip_moe_shared_workspace_bytes(int64_t tokens, int64_t hidden, int64_t inter) {
    if (tokens < 0 || hidden <= 0 || inter <= 0) return -1;
    return (int64_t)gollek::moe_shared_layout(tokens, hidden, inter).total;
}

int32_t gollek_hip_moe_shared_expert_device(gollek_hip_weight *gate, gollek_hip_weight *up,
                                            gollek_hip_weight *down, const float *gate_inp, const float *x,
                                            int64_t tokens, float *out, void *workspace,
                                            int64_t workspace_bytes, void *stream, char *err,
                                            size_t err_len) {
    MoeShape sh;
    int32_t rc = check_moe(gate, up, down, 1, tokens, 1, &sh, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    if (tokens == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    if (x == nullptr || out == nullptr || workspace == nullptr)
        return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "shared expert buffers");
    const int64_t need = gollek_hip_moe_shared_workspace_bytes(tokens, sh.H, sh.I);
    if (workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len,
                    "Workspace of %lld bytes (256-byte aligned) needed, got %lld",
                    (long long)need, (long long)workspace_bytes);
    const hipError_t e = gollek::launch_moe_shared(
        gate->type_id, up->type_id, down->type_id, gate->data, up->data, down->data, gate->row_bytes,
        up->row_bytes, down->row_bytes, sh.H, sh.I, x, gate_inp, (int)tokens, out,
        static_cast<uint8_t *>(workspace), static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "shared expert launch", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_moe_shared_expert(gollek_hip_weight *gate, gollek_hip_weight *up,
                                     gollek_hip_weight *down, const float *gate_inp, const float *x,
                                     int64_t tokens, float *out, int64_t out_len, char *err,
                                     size_t err_len) {
    MoeShape sh;
    int32_t rc = check_moe(gate, up, down, 1, tokens, 1, &sh, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    if (x == nullptr || out == nullptr)
        return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "shared expert buffers");
    if (out_len < tokens * sh.H)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Output length %lld is smaller than %lld x %d",
                    (long long)out_len, (long long)tokens, sh.H);
    if (tokens == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    std::lock_guard<std::mutex> lock(gate->mu);
    rc = use_device(gate->device, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    const size_t xn = (size_t)(tokens * sh.H) * 4, gn = (size_t)sh.H * 4;
    const size_t xb = align_up(xn, 256), gb = align_up(gn, 256);
    const size_t ws = (size_t)gollek_hip_moe_shared_workspace_bytes(tokens, sh.H, sh.I);
    rc = ensure_staging(gate, 2 * xb + gb + ws, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    uint8_t *base = gate->staging;
    float *d_x = reinterpret_cast<float *>(base);
    float *d_out = reinterpret_cast<float *>(base + xb);
    float *d_gi = gate_inp != nullptr ? reinterpret_cast<float *>(base + 2 * xb) : nullptr;
    hipStream_t s = gate->stream;
    hipError_t e = hipMemcpyAsync(d_x, x, xn, hipMemcpyHostToDevice, s);
    if (e == hipSuccess) e = hipMemcpyAsync(d_out, out, xn, hipMemcpyHostToDevice, s);
    if (e == hipSuccess && d_gi != nullptr) e = hipMemcpyAsync(d_gi, gate_inp, gn, hipMemcpyHostToDevice, s);
    if (e == hipSuccess)
        e = gollek::launch_moe_shared(gate->type_id, up->type_id, down->type_id, gate->data, up->data, down->data,
                                      gate->row_bytes, up->row_bytes, down->row_bytes, sh.H, sh.I, d_x, d_gi,
                                      (int)tokens, d_out, base + 2 * xb + gb, s);
    if (e == hipSuccess) e = hipMemcpyAsync(out, d_out, xn, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "shared expert", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

}  // extern "C"

// ---- MoE router ---------------------------------------------------------

namespace {

int32_t check_router(int64_t tokens, int64_t n_experts, int64_t top_k, int32_t scoring, char *err,
                     size_t err_len) {
    if (scoring != GOLLEK_HIP_ROUTER_SOFTMAX && scoring != GOLLEK_HIP_ROUTER_SIGMOID)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Unknown router scoring %d", scoring);
    if (n_experts <= 0 || n_experts > kRouterMaxExperts || top_k <= 0 || top_k > kRouterMaxExperts)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len,
                    "Router needs 1 <= experts, top_k <= %d (got %lld, %lld)", (int)kRouterMaxExperts,
                    (long long)n_experts, (long long)top_k);
    if (tokens < 0 || tokens > (1 << 24) || tokens * top_k > (1 << 24) ||
        tokens * n_experts > (1LL << 30))
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Invalid tokens %lld / top_k %lld",
                    (long long)tokens, (long long)top_k);
    return GOLLEK_HIP_OK;
}

}  // namespace

extern "C" {

int32_t gollek_hip_moe_select_topk_device(const float *logits, int64_t tokens, int64_t n_experts,
                                          int64_t top_k, int32_t scoring, int32_t *ids,
                                          float *weights, void *stream, char *err,
                                          size_t err_len) {
    int32_t rc = check_router(tokens, n_experts, top_k, scoring, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    if (tokens == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    if (logits == nullptr || ids == nullptr || weights == nullptr)
        return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "router buffers");
    const hipError_t e =
        gollek::launch_moe_topk(logits, (int)tokens, (int)n_experts, (int)top_k,
                                scoring == GOLLEK_HIP_ROUTER_SIGMOID, ids, weights,
                                static_cast<hipStream_t>(stream));
    if (e != hipSuccess) return hip_fail(e, "router launch", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_moe_select_topk(const float *logits, int64_t tokens, int64_t n_experts,
                                   int64_t top_k, int32_t scoring, int32_t *ids, float *weights,
                                   char *err, size_t err_len) {
    int32_t rc = check_router(tokens, n_experts, top_k, scoring, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    if (logits == nullptr || ids == nullptr || weights == nullptr)
        return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "router buffers");
    if (tokens == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    int device = 0;
    hipError_t e = hipGetDevice(&device);
    if (e != hipSuccess) return hip_fail(e, "hipGetDevice", err, err_len);
    rc = use_device(device, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    const size_t lb = align_up((size_t)(tokens * n_experts) * 4, 256);
    const size_t rb = align_up((size_t)(tokens * top_k) * 4, 256);
    uint8_t *buf = nullptr;
    e = hipMalloc(reinterpret_cast<void **>(&buf), lb + 2 * rb);
    if (e != hipSuccess) return hip_fail(e, "hipMalloc(router)", err, err_len);
    float *d_l = reinterpret_cast<float *>(buf);
    int32_t *d_ids = reinterpret_cast<int32_t *>(buf + lb);
    float *d_w = reinterpret_cast<float *>(buf + lb + rb);
    e = hipMemcpy(d_l, logits, (size_t)(tokens * n_experts) * 4, hipMemcpyHostToDevice);
    if (e == hipSuccess)
        e = gollek::launch_moe_topk(d_l, (int)tokens, (int)n_experts, (int)top_k,
                                    scoring == GOLLEK_HIP_ROUTER_SIGMOID, d_ids, d_w, nullptr);
    if (e == hipSuccess) e = hipMemcpy(ids, d_ids, (size_t)(tokens * top_k) * 4, hipMemcpyDeviceToHost);
    if (e == hipSuccess) e = hipMemcpy(weights, d_w, (size_t)(tokens * top_k) * 4, hipMemcpyDeviceToHost);
    (void)hipFree(buf);
    if (e != hipSuccess) return hip_fail(e, "router", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_moe_block_device(gollek_hip_weight *gate, gollek_hip_weight *up,
                                    gollek_hip_weight *down, int64_t n_experts, const float *x,
                                    const float *logits, int64_t tokens, int64_t top_k,
                                    int32_t scoring, int32_t *ids, float *weights, float *out,
                                    void *workspace, int64_t workspace_bytes, void *stream,
                                    char *err, size_t err_len) {
    int32_t rc = check_router(tokens, n_experts, top_k, scoring, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    MoeShape sh;
    rc = check_moe(gate, up, down, n_experts, tokens, top_k, &sh, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    if (tokens == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    if (x == nullptr || logits == nullptr || ids == nullptr || weights == nullptr || out == nullptr ||
        workspace == nullptr)
        return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "MoE block buffers");
    const int64_t need = gollek_hip_moe_workspace_bytes(tokens, top_k, sh.H, sh.I, sh.E);
    if (workspace_bytes < need || (reinterpret_cast<uintptr_t>(workspace) & 255u) != 0)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len,
                    "Workspace of %lld bytes (256-byte aligned) needed, got %lld",
                    (long long)need, (long long)workspace_bytes);
    const hipStream_t s = static_cast<hipStream_t>(stream);
    hipError_t e = gollek::launch_moe_topk(logits, (int)tokens, sh.E, (int)top_k,
                                           scoring == GOLLEK_HIP_ROUTER_SIGMOID, ids, weights, s);
    if (e == hipSuccess)
        e = moe_launch(sh, gate, up, down, x, ids, weights, tokens, top_k, out,
                       static_cast<uint8_t *>(workspace), s);
    if (e != hipSuccess) return hip_fail(e, "moe block launch", err, err_len);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_moe_block(gollek_hip_weight *gate, gollek_hip_weight *up,
                             gollek_hip_weight *down, int64_t n_experts, const float *x,
                             int64_t tokens, const float *logits, int64_t top_k, int32_t scoring,
                             float *out, int64_t out_len, char *err, size_t err_len) {
    int32_t rc = check_router(tokens, n_experts, top_k, scoring, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    MoeShape sh;
    rc = check_moe(gate, up, down, n_experts, tokens, top_k, &sh, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    if (x == nullptr || logits == nullptr || out == nullptr)
        return fail(GOLLEK_HIP_ERR_NULL, err, err_len, "MoE block buffers");
    if (out_len < tokens * sh.H)
        return fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Output length %lld is smaller than %lld x %d",
                    (long long)out_len, (long long)tokens, sh.H);
    if (tokens == 0) {
        ok(err, err_len);
        return GOLLEK_HIP_OK;
    }
    std::lock_guard<std::mutex> lock(gate->mu);
    rc = use_device(gate->device, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    const size_t xb = align_up((size_t)(tokens * sh.H) * 4, 256);
    const size_t lb = align_up((size_t)(tokens * sh.E) * 4, 256);
    const size_t rb = align_up((size_t)(tokens * top_k) * 4, 256);
    const size_t ws = (size_t)gollek_hip_moe_workspace_bytes(tokens, top_k, sh.H, sh.I, sh.E);
    rc = ensure_staging(gate, 2 * xb + lb + 2 * rb + ws, err, err_len);
    if (rc != GOLLEK_HIP_OK) return rc;
    uint8_t *base = gate->staging;
    float *d_x = reinterpret_cast<float *>(base);
    float *d_out = reinterpret_cast<float *>(base + xb);
    float *d_l = reinterpret_cast<float *>(base + 2 * xb);
    int32_t *d_ids = reinterpret_cast<int32_t *>(base + 2 * xb + lb);
    float *d_w = reinterpret_cast<float *>(base + 2 * xb + lb + rb);
    uint8_t *d_ws = base + 2 * xb + lb + 2 * rb;
    hipStream_t s = gate->stream;
    const size_t xn = (size_t)(tokens * sh.H) * 4, ln = (size_t)(tokens * sh.E) * 4;
    // Pinned staging laid out as the device buffer (x | out | logits): the
    // inputs go up in one copy and the expert passes store `out` into it.
    uint8_t *hs = host_staging(gate, 2 * xb + lb);
    hipError_t e = hipSuccess;
    if (hs != nullptr) {
        std::memcpy(hs, x, xn);
        std::memcpy(hs + 2 * xb, logits, ln);
        e = pull_staging(d_x, hs, xn, s, 2 * xb - xn, lb);
    } else {
        e = hipMemcpyAsync(d_x, x, xn, hipMemcpyHostToDevice, s);
        if (e == hipSuccess) e = hipMemcpyAsync(d_l, logits, ln, hipMemcpyHostToDevice, s);
    }
    float *k_out = hs != nullptr ? reinterpret_cast<float *>(hs + xb) : d_out;
    if (e == hipSuccess)
        e = gollek::launch_moe_topk(d_l, (int)tokens, sh.E, (int)top_k,
                                    scoring == GOLLEK_HIP_ROUTER_SIGMOID, d_ids, d_w, s);
    if (e == hipSuccess)
        e = moe_launch(sh, gate, up, down, d_x, d_ids, d_w, tokens, top_k, k_out, d_ws, s);
    if (e == hipSuccess && hs == nullptr) e = hipMemcpyAsync(out, d_out, xn, hipMemcpyDeviceToHost, s);
    if (e == hipSuccess) e = hipStreamSynchronize(s);
    if (e != hipSuccess) return hip_fail(e, "moe block", err, err_len);
    if (hs != nullptr) std::memcpy(out, hs + xb, xn);
    ok(err, err_len);
    return GOLLEK_HIP_OK;
}

}  // extern "C"

namespace gollek {

void record_status(int32_t code, const char *message) {
    g_last_status = code;
    try {
        g_last_error = message != nullptr ? message : "";
    } catch (const std::bad_alloc &) {
        g_last_error.clear();
    }
}

gollek_hip_weight *weight_alloc_owned(int32_t type_id, int64_t rows, int64_t cols, int64_t row_bytes,
                                      char *err, size_t err_len) {
    gollek_hip_weight *w = make_weight(type_id, rows, cols, row_bytes, err, err_len);
    if (w == nullptr) return nullptr;
    const size_t bytes = (size_t)rows * (size_t)row_bytes;
    if (bytes > 0) {
        const hipError_t e = hipMalloc(reinterpret_cast<void **>(&w->data), bytes);
        if (e != hipSuccess) {
            hip_fail(e, "hipMalloc(weight)", err, err_len);
            gollek_hip_weight_free(w);
            return nullptr;
        }
    }
    w->owned = true;
    return w;
}

uint8_t *weight_data(gollek_hip_weight *w) { return w->data; }

}  // namespace gollek
