// gguf_file.hip -- GGUF files: read-only mmap, header / metadata / tensor-info
// parse, and the one-time upload of a tensor's bytes to a device handle.
//
// Replaces the reference's loader (GC/ = runner/gguf/gollek-gguf-core/src/main/
// java/tech/kayys/gollek/gguf/): GC/loader/GGUFReader.java:28-37 maps the
// whole file read-only; GC/loader/GGUFParser.java:17-105 reads the header
// ("GGUF", version, tensor count, KV count), skips over the metadata values
// (keeping general.alignment, default 32), reads the tensor infos (name,
// dims, type, offset; size from GC/core/GgmlType.java:70-81) and aligns the
// data start; RT/GgufTensorData.java:97-104 (RT/ = GC/runtime/) slices a
// tensor's bytes at dataStart + offset after a range check.  Little-endian
// fields at any alignment, like the reference's unaligned cursor
// (GC/loader/GGUFReader.java:54-147).  Malformed or truncated files are
// rejected with an error instead of reading past the mapping.
//
// Parsing needs no GPU.  The upload copies the mapped bytes through a pinned
// staging buffer in double-buffered chunks (the copy engine reads pinned
// memory at full speed; registering the mapping itself is not used).
#include <errno.h>
#include <fcntl.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <unistd.h>

#include <algorithm>
#include <mutex>
#include <new>
#include <thread>
#include <string>
#include <unordered_map>
#include <vector>

#include "gguf_kernels.hpp"
#include "gollek_hip.h"

namespace {

// (block elements, bytes per block) by ggml type id, GC/core/GgmlType.java:9-52.
// Ids without an entry or with 0 / 0 (runtime-repacked layouts) cannot be
// loaded from GGUF data.
struct TypeGeom {
    int block, bytes;
};
constexpr TypeGeom kTypes[] = {
    {1, 4},    {1, 2},    {32, 18},  {32, 20},  {0, 0},    {0, 0},    {32, 22},  {32, 24},   // 0-7
    {32, 34},  {32, 36},  {256, 84}, {256, 110}, {256, 144}, {256, 176}, {256, 210}, {256, 292},  // 8-15
    {256, 66}, {256, 74}, {256, 98}, {256, 50}, {32, 18},  {256, 110}, {256, 82}, {256, 136},  // 16-23
    {1, 1},    {1, 2},    {1, 4},    {1, 8},    {1, 8},    {256, 56}, {1, 2},    {0, 0},      // 24-31
    {0, 0},    {0, 0},    {256, 54}, {256, 66}, {0, 0},    {0, 0},    {0, 0},    {32, 17},    // 32-39
    {64, 36},  {128, 18},                                                                     // 40-41
};
constexpr int kNumTypes = sizeof(kTypes) / sizeof(kTypes[0]);

constexpr int kMaxDims = 8;
// Upload staging: up to kLanes host threads each copy every kLanes-th chunk
// of kSlotBytes from the mapped file into one of their two pinned slots and
// queue its DMA, so host copies run in parallel with each other and with the
// DMAs (one thread's copy alone moves ~10-20 GB/s).  64 MiB pinned in all.
constexpr int kLanes = 8;
constexpr size_t kSlotBytes = 4u << 20;

struct TensorInfo {
    std::string name;
    int32_t n_dims = 0;
    int64_t dims[kMaxDims] = {};
    int32_t type_id = 0;
    int64_t offset = 0, size = 0;
};

int32_t file_fail(int32_t code, char *err, size_t err_len, const char *fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    gollek::record_status(code, buf);
    if (err != nullptr && err_len > 0) {
        size_t n = strlen(buf);
        if (n >= err_len) n = err_len - 1;
        memcpy(err, buf, n);
        err[n] = '\0';
    }
    return code;
}

// Bounds-checked little-endian cursor over the mapping.
struct Cursor {
    const uint8_t *p;
    uint64_t size, pos = 0;
    bool ok = true;
    bool take(void *dst, uint64_t n) {
        if (!ok || n > size - pos) {
            ok = false;
            return false;
        }
        memcpy(dst, p + pos, n);
        pos += n;
        return true;
    }
    template <typename T>
    T get() {
        T v{};
        take(&v, sizeof(T));
        return v;
    }
    bool skip(uint64_t n) {
        if (!ok || n > size - pos) return ok = false;
        pos += n;
        return true;
    }
};

}  // namespace

struct gollek_hip_gguf {
    int fd = -1;
    uint8_t *map = nullptr;
    uint64_t size = 0;
    int32_t version = 0;
    int64_t n_kv = 0, alignment = 32, data_start = 0;
    std::vector<TensorInfo> tensors;
    std::unordered_map<std::string, int64_t> by_name;
    // upload resources, created at the first upload; uploads serialise on mu
    std::mutex mu;
    uint8_t *stage[kLanes][2] = {};
    hipStream_t stream = nullptr;
    hipEvent_t done[kLanes][2] = {};
};

namespace {

// Frees the upload stream, staging buffers and events (whichever exist)
// and clears their handles.
void release_staging(gollek_hip_gguf *f) {
    if (f->stream != nullptr) (void)hipStreamSynchronize(f->stream);
    for (int l = 0; l < kLanes; l++) {
        for (int i = 0; i < 2; i++) {
            if (f->done[l][i] != nullptr) (void)hipEventDestroy(f->done[l][i]);
            if (f->stage[l][i] != nullptr) (void)hipHostFree(f->stage[l][i]);
            f->done[l][i] = nullptr;
            f->stage[l][i] = nullptr;
        }
    }
    if (f->stream != nullptr) (void)hipStreamDestroy(f->stream);
    f->stream = nullptr;
}

void release(gollek_hip_gguf *f) {
    release_staging(f);
    if (f->map != nullptr) munmap(f->map, f->size);
    if (f->fd >= 0) close(f->fd);
    delete f;
}

// Skips one metadata value of `type` (GC/loader/GGUFParser.java:64-99);
// general.alignment is kept when its value is a number.  Returns 0 or a
// status code.
int32_t skip_value(Cursor &c, int32_t type, bool is_alignment, int64_t *alignment, int depth, char *err,
                   size_t err_len) {
    static const int fixed[] = {1, 1, 2, 2, 4, 4, 4, 1, 0, 0, 8, 8, 8};
    if (type < 0 || type > 12)
        return file_fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len, "Unsupported GGUF KV type: %d at pos %llu",
                         type, (unsigned long long)c.pos);
    if (type == 8) {  // string
        const int64_t len = c.get<int64_t>();
        if (c.ok && (len < 0 || len > 0x7FFFFFFF))
            return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Invalid string length: %lld", (long long)len);
        c.skip((uint64_t)len);
    } else if (type == 9) {  // array: element type, count, elements
        const int32_t et = c.get<int32_t>();
        const int64_t n = c.get<int64_t>();
        if (c.ok && (n < 0 || depth > 4))
            return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Invalid GGUF array (length %lld) at pos %llu",
                             (long long)n, (unsigned long long)c.pos);
        if (c.ok && et >= 0 && et <= 12 && et != 8 && et != 9) {
            const uint64_t bytes = (uint64_t)fixed[et] * (uint64_t)n;
            if ((uint64_t)n > c.size || !c.skip(bytes)) c.ok = false;
        } else {
            for (int64_t i = 0; i < n && c.ok; i++) {
                const int32_t rc = skip_value(c, et, false, nullptr, depth + 1, err, err_len);
                if (rc != GOLLEK_HIP_OK) return rc;
            }
        }
    } else {
        uint8_t v[8] = {};
        c.take(v, (uint64_t)fixed[type]);
        // The alignment is read as a 32-bit int whatever its numeric type
        // (the reference's Number.intValue(): low 32 bits of an integer,
        // saturating truncation of a float); a bool is not a number.
        if (is_alignment && c.ok && type != 7) {
            int64_t a = 0;
            double d = 0.0;
            switch (type) {
            case 0: a = v[0]; break;
            case 1: a = (int8_t)v[0]; break;
            case 2: { uint16_t t; memcpy(&t, v, 2); a = t; break; }
            case 3: { int16_t t; memcpy(&t, v, 2); a = t; break; }
            case 4: { uint32_t t; memcpy(&t, v, 4); a = t; break; }
            case 5: { int32_t t; memcpy(&t, v, 4); a = t; break; }
            case 6: { float t; memcpy(&t, v, 4); d = t; break; }
            case 12: memcpy(&d, v, 8); break;
            default: memcpy(&a, v, 8); break;
            }
            if (type == 6 || type == 12)
                a = d != d ? 0 : d >= 2147483647.0 ? 2147483647 : d <= -2147483648.0 ? -2147483648LL : (int64_t)d;
            else
                a = (int32_t)(uint32_t)(uint64_t)a;
            *alignment = a;
        }
    }
    return GOLLEK_HIP_OK;
}

int32_t parse(gollek_hip_gguf *f, char *err, size_t err_len) {
    Cursor c{f->map, f->size};
    char magic[4] = {};
    c.take(magic, 4);
    if (!c.ok || memcmp(magic, "GGUF", 4) != 0)
        return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Not a valid GGUF file");
    f->version = c.get<int32_t>();
    const int64_t n_tensors = c.get<int64_t>();
    f->n_kv = c.get<int64_t>();
    // Every metadata entry takes at least 12 bytes (key length, type, a value
    // of at least one byte less one) and every tensor info at least 24 (name
    // length, dimension count, type, offset), so counts the bytes left cannot
    // hold are rejected before anything is sized by them.
    const uint64_t left = c.ok ? c.size - c.pos : 0;
    if (c.ok && (n_tensors < 0 || f->n_kv < 0 || (uint64_t)f->n_kv > left / 12 ||
                 (uint64_t)n_tensors > (left - (uint64_t)f->n_kv * 12) / 24))
        return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Invalid GGUF counts: %lld tensors, %lld keys",
                         (long long)n_tensors, (long long)f->n_kv);
    for (int64_t i = 0; i < f->n_kv && c.ok; i++) {
        const int64_t klen = c.get<int64_t>();
        if (c.ok && (klen < 0 || klen > 0x7FFFFFFF))
            return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Invalid string length: %lld", (long long)klen);
        const bool is_alignment = c.ok && klen == 17 && klen <= (int64_t)(c.size - c.pos) &&
                                  memcmp(c.p + c.pos, "general.alignment", 17) == 0;
        c.skip((uint64_t)klen);
        const int32_t type = c.get<int32_t>();
        if (!c.ok) break;
        if (is_alignment && (type == 7 || type == 8 || type == 9))
            return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "general.alignment is not a number (KV type %d)",
                             type);
        const int32_t rc = skip_value(c, type, is_alignment, &f->alignment, 0, err, err_len);
        if (rc != GOLLEK_HIP_OK) return rc;
    }
    for (int64_t i = 0; i < n_tensors && c.ok; i++) {
        TensorInfo t;
        const int64_t nlen = c.get<int64_t>();
        if (c.ok && (nlen < 0 || nlen > 0x7FFFFFFF))
            return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Invalid string length: %lld", (long long)nlen);
        if (c.ok && (uint64_t)nlen <= c.size - c.pos) t.name.assign((const char *)c.p + c.pos, (size_t)nlen);
        c.skip((uint64_t)nlen);
        t.n_dims = c.get<int32_t>();
        if (c.ok && (t.n_dims < 0 || t.n_dims > kMaxDims))
            return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Tensor %s has %d dimensions", t.name.c_str(),
                             t.n_dims);
        // Element count; a negative dimension or a product beyond int64 is
        // rejected (a zero dimension makes the count zero).
        int64_t elements = 1;
        bool overflow = false, zero = false;
        for (int d = 0; d < t.n_dims; d++) {
            t.dims[d] = c.get<int64_t>();
            if (t.dims[d] < 0) overflow = true;
            else if (t.dims[d] == 0) zero = true;
            else if (elements > INT64_MAX / t.dims[d]) overflow = true;
            else elements *= t.dims[d];
        }
        if (zero) elements = 0;
        t.type_id = c.get<int32_t>();
        t.offset = c.get<int64_t>();
        if (!c.ok) break;
        if (overflow)
            return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Tensor %s has an invalid shape", t.name.c_str());
        const bool known = t.type_id >= 0 && t.type_id < kNumTypes && kTypes[t.type_id].block > 0;
        if (!known || elements % kTypes[t.type_id].block != 0)
            return file_fail(GOLLEK_HIP_ERR_UNSUPPORTED, err, err_len,
                             "Unsupported or misaligned GGUF tensor type %d with %lld element(s)", t.type_id,
                             (long long)elements);
        t.size = elements / kTypes[t.type_id].block * kTypes[t.type_id].bytes;
        f->by_name.emplace(t.name, (int64_t)f->tensors.size());
        f->tensors.push_back(std::move(t));
    }
    if (!c.ok)
        return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Truncated GGUF file (%llu bytes)",
                         (unsigned long long)f->size);
    if (f->alignment <= 0)
        return file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Invalid general.alignment %lld",
                         (long long)f->alignment);
    const int64_t pos = (int64_t)c.pos;
    f->data_start = pos + (f->alignment - pos % f->alignment) % f->alignment;
    return GOLLEK_HIP_OK;
}

}  // namespace

extern "C" {

gollek_hip_gguf *gollek_hip_gguf_open(const char *path, char *err, size_t err_len) {
    if (path == nullptr) {
        file_fail(GOLLEK_HIP_ERR_NULL, err, err_len, "path");
        return nullptr;
    }
    gollek_hip_gguf *f = new (std::nothrow) gollek_hip_gguf();
    if (f == nullptr) {
        file_fail(GOLLEK_HIP_ERR_NOMEM, err, err_len, "out of host memory");
        return nullptr;
    }
    f->fd = open(path, O_RDONLY | O_CLOEXEC);
    struct stat st;
    if (f->fd < 0 || fstat(f->fd, &st) != 0) {
        file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Cannot open %s: %s", path, strerror(errno));
        release(f);
        return nullptr;
    }
    f->size = (uint64_t)st.st_size;
    if (f->size > 0) {
        void *m = mmap(nullptr, f->size, PROT_READ, MAP_PRIVATE, f->fd, 0);
        if (m == MAP_FAILED) {
            file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Cannot map %s: %s", path, strerror(errno));
            release(f);
            return nullptr;
        }
        f->map = static_cast<uint8_t *>(m);
    }
    int32_t rc;
    try {
        rc = parse(f, err, err_len);
    } catch (const std::bad_alloc &) {  // the tensor table outgrew host memory
        rc = file_fail(GOLLEK_HIP_ERR_NOMEM, err, err_len, "Out of host memory parsing %s", path);
    }
    if (rc != GOLLEK_HIP_OK) {
        release(f);
        return nullptr;
    }
    gollek::record_status(GOLLEK_HIP_OK, "");
    if (err != nullptr && err_len > 0) err[0] = '\0';
    return f;
}

void gollek_hip_gguf_close(gollek_hip_gguf *f) {
    if (f != nullptr) release(f);
}

int32_t gollek_hip_gguf_info(const gollek_hip_gguf *f, int32_t *version, int64_t *n_tensors, int64_t *n_kv,
                             int64_t *alignment, int64_t *data_start, int64_t *file_bytes) {
    if (f == nullptr) return GOLLEK_HIP_ERR_NULL;
    if (version) *version = f->version;
    if (n_tensors) *n_tensors = (int64_t)f->tensors.size();
    if (n_kv) *n_kv = f->n_kv;
    if (alignment) *alignment = f->alignment;
    if (data_start) *data_start = f->data_start;
    if (file_bytes) *file_bytes = (int64_t)f->size;
    return GOLLEK_HIP_OK;
}

int32_t gollek_hip_gguf_tensor(const gollek_hip_gguf *f, int64_t index, char *name, size_t name_len,
                               int32_t *type_id, int32_t *n_dims, int64_t *dims, int64_t *offset,
                               int64_t *size_bytes) {
    if (f == nullptr) return GOLLEK_HIP_ERR_NULL;
    if (index < 0 || index >= (int64_t)f->tensors.size()) return GOLLEK_HIP_ERR_ARG;
    const TensorInfo &t = f->tensors[(size_t)index];
    if (name != nullptr && name_len > 0) {
        const size_t n = t.name.size() < name_len - 1 ? t.name.size() : name_len - 1;
        memcpy(name, t.name.data(), n);
        name[n] = '\0';
    }
    if (type_id) *type_id = t.type_id;
    if (n_dims) *n_dims = t.n_dims;
    if (dims)
        for (int d = 0; d < kMaxDims; d++) dims[d] = d < t.n_dims ? t.dims[d] : 1;
    if (offset) *offset = t.offset;
    if (size_bytes) *size_bytes = t.size;
    return GOLLEK_HIP_OK;
}

int64_t gollek_hip_gguf_find(const gollek_hip_gguf *f, const char *name) {
    if (f == nullptr || name == nullptr) return -1;
    try {
        const auto it = f->by_name.find(name);
        return it == f->by_name.end() ? -1 : it->second;
    } catch (const std::bad_alloc &) {  // the key string could not be built
        return -1;
    }
}

gollek_hip_weight *gollek_hip_gguf_upload(gollek_hip_gguf *f, int64_t index, char *err, size_t err_len) {
    if (f == nullptr) {
        file_fail(GOLLEK_HIP_ERR_NULL, err, err_len, "file");
        return nullptr;
    }
    if (index < 0 || index >= (int64_t)f->tensors.size()) {
        file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Tensor index %lld is outside [0, %lld)", (long long)index,
                  (long long)f->tensors.size());
        return nullptr;
    }
    const TensorInfo &t = f->tensors[(size_t)index];
    // RT/GgufTensorData.java:97-104: the bytes must lie inside the file.
    const int64_t room = (int64_t)f->size - f->data_start;  // bytes after the data start (may be < 0)
    if (t.offset < 0 || t.offset > room || t.size > room - t.offset) {
        file_fail(GOLLEK_HIP_ERR_ARG, err, err_len, "Tensor data range is outside model segment: %s",
                  t.name.c_str());
        return nullptr;
    }
    // Matrix view (RT/GgufTensorOps.java:621-630): columns = dims[0], rows =
    // the product of the other dimensions.
    const int64_t cols = t.n_dims > 0 ? t.dims[0] : 1;
    const int64_t elements = t.size / kTypes[t.type_id].bytes * kTypes[t.type_id].block;
    const int64_t rows = cols > 0 ? elements / cols : 0;
    const int64_t row_bytes = cols / kTypes[t.type_id].block * kTypes[t.type_id].bytes;
    // Validation (type, shape) and the device buffer; the bytes follow.
    gollek_hip_weight *w = gollek::weight_alloc_owned(t.type_id, rows, cols, row_bytes, err, err_len);
    if (w == nullptr) return nullptr;
    uint8_t *dst = gollek::weight_data(w);
    std::lock_guard<std::mutex> lock(f->mu);
    hipError_t e = hipSuccess;
    // The stream, the pinned slots and their events are set up together at
    // the first upload: if any of them fails, all are released, so a later
    // call sets them up again instead of using a partial set.
    if (f->stream == nullptr || f->stage[kLanes - 1][1] == nullptr || f->done[kLanes - 1][1] == nullptr) {
        release_staging(f);
        e = hipStreamCreateWithFlags(&f->stream, hipStreamNonBlocking);
        for (int l = 0; l < kLanes; l++) {
            for (int i = 0; i < 2 && e == hipSuccess; i++) {
                e = hipHostMalloc(reinterpret_cast<void **>(&f->stage[l][i]), kSlotBytes, hipHostMallocDefault);
                if (e == hipSuccess) e = hipEventCreateWithFlags(&f->done[l][i], hipEventDisableTiming);
            }
        }
        if (e != hipSuccess) release_staging(f);
    }
    // Chunk k (kSlotBytes from offset k * kSlotBytes) belongs to lane
    // k % lanes and goes through that lane's slot (k / lanes) % 2, once the
    // DMA that last read the slot has finished.  All DMAs share f->stream;
    // an event recorded after a lane's DMA may also cover other lanes' DMAs
    // queued before it, which only makes the wait longer.
    const uint8_t *src = f->map + f->data_start + t.offset;
    const int64_t chunks = (t.size + (int64_t)kSlotBytes - 1) / (int64_t)kSlotBytes;
    const unsigned hw = std::thread::hardware_concurrency();
    const int lanes = (int)std::min<int64_t>(std::min<int64_t>(kLanes, hw == 0 ? 1 : hw), std::max<int64_t>(chunks, 1));
    hipError_t lane_err[kLanes];
    auto lane = [&](int l) {
        hipError_t le = hipSuccess;
        for (int64_t k = l, j = 0; k < chunks && le == hipSuccess; k += lanes, j++) {
            const int b = (int)(j & 1);
            const int64_t off = k * (int64_t)kSlotBytes;
            const size_t n = (size_t)std::min<int64_t>((int64_t)kSlotBytes, t.size - off);
            if (j >= 2) le = hipEventSynchronize(f->done[l][b]);
            if (le != hipSuccess) break;
            memcpy(f->stage[l][b], src + off, n);
            le = hipMemcpyAsync(dst + off, f->stage[l][b], n, hipMemcpyHostToDevice, f->stream);
            if (le == hipSuccess) le = hipEventRecord(f->done[l][b], f->stream);
        }
        lane_err[l] = le;
    };
    if (e == hipSuccess) {
        // Lanes 1.. on their own threads; the calling thread runs lane 0 and
        // then any lane whose thread could not be started (fixed arrays: no
        // allocation that could throw out of this entry point).
        std::thread th[kLanes];
        bool started[kLanes] = {};
        for (int l = 1; l < lanes; l++) {
            try {
                th[l] = std::thread(lane, l);
                started[l] = true;
            } catch (...) {
            }
        }
        lane(0);
        for (int l = 1; l < lanes; l++)
            if (!started[l]) lane(l);
        for (int l = 1; l < lanes; l++)
            if (started[l]) th[l].join();
        for (int l = 0; l < lanes && e == hipSuccess; l++) e = lane_err[l];
        // Wait for every queued DMA, also after an error in one lane.
        const hipError_t es = hipStreamSynchronize(f->stream);
        if (e == hipSuccess) e = es;
    }
    if (e != hipSuccess) {
        file_fail(e == hipErrorOutOfMemory ? GOLLEK_HIP_ERR_NOMEM : GOLLEK_HIP_ERR_DEVICE, err, err_len,
                  "GGUF upload of %s failed: %s", t.name.c_str(), hipGetErrorString(e));
        gollek_hip_weight_free(w);
        return nullptr;
    }
    gollek::record_status(GOLLEK_HIP_OK, "");
    if (err != nullptr && err_len > 0) err[0] = '\0';
    return w;
}

}  // extern "C"
