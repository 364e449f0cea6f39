// capi.hip -- library-level C ABI: version, last error, device query, host
// structural check, and the internals declared in common.hpp.
#include <cstdarg>
#include <map>
#include <mutex>
#include <utility>
#include <vector>

#include "common.hpp"

namespace jlust {

static thread_local std::string g_last_error;

int fail(int code, const char *fmt, ...)
{
    char buf[1024];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    try {
        g_last_error = buf;
    } catch (const std::bad_alloc &) {
        g_last_error.clear();   // the status code still reports the failure
    }
    return code;
}

void clear_error() { g_last_error.clear(); }

int hip_fail(hipError_t e, const char *what)
{
    if (e == hipErrorOutOfMemory)
        return fail(JLUST_STATUS_OUT_OF_MEMORY, "%s: %s", what, hipGetErrorString(e));
    if (e == hipErrorNoDevice || e == hipErrorInvalidDevice)
        return fail(JLUST_STATUS_NO_DEVICE, "%s: %s", what, hipGetErrorString(e));
    return fail(JLUST_STATUS_HIP_ERROR, "%s: %s", what, hipGetErrorString(e));
}

int require_device(int *device_out)
{
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count <= 0) {
        (void)hipGetLastError();
        return fail(JLUST_STATUS_NO_DEVICE, "no HIP device available (%s)",
                    e == hipSuccess ? "device count is 0" : hipGetErrorString(e));
    }
    int dev = 0;
    JLUST_HIP_TRY(hipGetDevice(&dev));
    if (device_out) *device_out = dev;
    return JLUST_STATUS_SUCCESS;
}

int check_launch(const char *kernel)
{
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return hip_fail(e, kernel);
    return JLUST_STATUS_SUCCESS;
}

int check_origin(int32_t origin)
{
    if (origin != 0 && origin != 1)
        return fail(JLUST_STATUS_INDEX_ORIGIN,
                    "index origin must be 0 (ZeroBased) or 1 (OneBased), got %d", origin);
    return JLUST_STATUS_SUCCESS;
}

// ------------------------------------------------------------------ devices

static std::mutex g_dev_mu;
static std::map<int, DeviceInfo> g_dev;

const DeviceInfo &device_info(int device)
{
    std::lock_guard<std::mutex> lk(g_dev_mu);
    auto it = g_dev.find(device);
    if (it != g_dev.end()) return it->second;
    DeviceInfo info;
    hipDeviceProp_t p;
    if (hipGetDeviceProperties(&p, device) == hipSuccess) {
        info.cu_count = p.multiProcessorCount;
        info.wave_size = p.warpSize;
        info.lds_per_block = p.sharedMemPerBlock;
        snprintf(info.arch, sizeof info.arch, "%s", p.gcnArchName);
    }
    return g_dev.emplace(device, info).first->second;
}

// ------------------------------------------------------------------ scratch

struct ScratchBuf {
    void *ptr = nullptr;
    size_t bytes = 0;
};
static std::mutex g_scratch_mu;
static std::map<std::pair<int, jlust_stream_t>, ScratchBuf> g_scratch;
// Buffers outgrown by a later call.  They are kept until the process ends:
// work already queued may still read them, and so may any HIP graph that
// captured a call on that stream and is replayed later.  Growth is by at
// least a quarter, so the kept buffers stay within a few times the largest.
static std::vector<void *> g_scratch_retired;

int scratch(jlust_stream_t stream, size_t bytes, void **out)
{
    int dev = 0;
    int st = require_device(&dev);
    if (st) return st;
    return host_guard("scratch", [&]() -> int {
        std::lock_guard<std::mutex> lk(g_scratch_mu);
        ScratchBuf &b = g_scratch[{dev, stream}];
        if (b.bytes < bytes) {
            const size_t want = bytes + bytes / 4 + 4096;
            if (b.ptr) g_scratch_retired.reserve(g_scratch_retired.size() + 1);   // before the hipMalloc
            void *p = nullptr;
            JLUST_HIP_TRY(hipMalloc(&p, want));
            if (b.ptr) g_scratch_retired.push_back(b.ptr);
            b.ptr = p;
            b.bytes = want;
        }
        *out = b.ptr;
        return JLUST_STATUS_SUCCESS;
    });
}

}  // namespace jlust

using namespace jlust;

extern "C" int jlust_hip_version(void) { return JLUST_HIP_ABI_VERSION; }

extern "C" int jlust_hip_preload(jlust_stream_t stream)
{
    clear_error();
    if (int st = require_device(nullptr)) return st;
    hipStream_t s = (hipStream_t)stream;
    for (int (*f)() : {preload_spmv, preload_spmm, preload_sddmm, preload_bsr, preload_coo_spmv, preload_coo_csc,
                       preload_assemble, preload_dcsr, preload_fn, preload_periodic, preload_scan})
        if (int st = f()) return st;
    for (int (*f)(hipStream_t) : {preload_binned, preload_coo_plan, preload_convert})
        if (int st = f(s)) return st;
    return JLUST_STATUS_SUCCESS;
}

extern "C" const char *jlust_hip_last_error(void) { return g_last_error.c_str(); }

extern "C" int jlust_hip_device_arch(char *buf, size_t len)
{
    clear_error();
    if (!buf || len == 0) return fail(JLUST_STATUS_INVALID_ARGUMENT, "device_arch: empty buffer");
    int dev = 0;
    int st = require_device(&dev);
    if (st) return st;
    snprintf(buf, len, "%s", device_info(dev).arch);
    return JLUST_STATUS_SUCCESS;
}

extern "C" int jlust_hip_check_csr(int64_t m, int64_t n, int64_t nnz, int32_t origin,
                                   const int32_t *rowptr, const int32_t *colind,
                                   int require_sorted)
{
    clear_error();
    if (m < 0 || n < 0 || nnz < 0)
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "check_csr: negative extent");
    if (int st = check_origin(origin)) return st;
    if (!rowptr || bad_ptr(colind, nnz))
        return fail(JLUST_STATUS_INVALID_ARGUMENT, "check_csr: null buffer");
    if (rowptr[0] != origin)
        return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                    "rowptr[0] = %d, expected the origin %d", rowptr[0], origin);
    if ((int64_t)rowptr[m] - origin != nnz)
        return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                    "rowptr[m] - origin = %lld, expected nnz = %lld",
                    (long long)rowptr[m] - origin, (long long)nnz);
    for (int64_t i = 0; i < m; ++i) {
        int64_t lo = (int64_t)rowptr[i] - origin, hi = (int64_t)rowptr[i + 1] - origin;
        if (hi < lo)
            return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                        "rowptr decreases at row %lld", (long long)i);
        for (int64_t p = lo; p < hi; ++p) {
            int64_t c = (int64_t)colind[p] - origin;
            if (c < 0 || c >= n)
                return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                            "column index %d at position %lld is outside [%d, %lld)",
                            colind[p], (long long)p, origin, (long long)(n + origin));
            if (require_sorted && p > lo && colind[p] <= colind[p - 1])
                return fail(JLUST_STATUS_NONCANONICAL_STORAGE,
                            "row %lld: column indices not strictly increasing at position %lld",
                            (long long)i, (long long)p);
        }
    }
    return JLUST_STATUS_SUCCESS;
}
