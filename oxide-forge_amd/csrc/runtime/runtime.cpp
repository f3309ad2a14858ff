// runtime.cpp -- implementation of the C ABI in include/oxforge.h.
//
// Replaces the cuda-oxide routing of the reference (src/cuda.rs,
// src/cuda/runtime.rs, src/cuda/span.rs): a HIP device context, a primary
// non-blocking stream, extra streams joined by events, an exact-size buffer
// pool, and kernel launches by name from the gfx950 code object through
// hipModuleLaunchKernel.  Kernel instances are chosen here from shape and
// alignment (the reference chooses its launch geometry in the container
// layer, e.g. matrix.rs:133-176 and norm.rs:8-24).
#include "oxforge.h"
#include "noalloc_scratch.h"

#include <hip/hip_runtime_api.h>
#include <dlfcn.h>

#include <algorithm>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <unordered_map>
#include <vector>

namespace {

thread_local std::string g_last_error;

forge_status fail(forge_status st, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return st;
}

#define HIP_TRY(expr)                                                          \
    do {                                                                       \
        hipError_t e_ = (expr);                                                \
        if (e_ != hipSuccess)                                                  \
            return fail(FORGE_EHIP, "%s failed: %s", #expr, hipGetErrorString(e_)); \
    } while (0)

#define FORGE_TRY(expr)                                                        \
    do {                                                                       \
        forge_status s_ = (expr);                                              \
        if (s_ != FORGE_OK) return s_;                                         \
    } while (0)

// Must match forge::GemmArgs in csrc/kernels/gemm.hpp.
struct GemmArgs {
    const float* A;
    const float* B;
    float* C;
    int M, N, K;
    long long lda, ldb, ldc;
    float alpha;
    const float* bias;
    const float* residual;
    const float* aux;
    float* pre_out;
    int act;
    int aux_act;
    int update;
    float update_scale;
    const float* row_part;
    const float* row_d;
    int row_parts, row_n;
    float row_eps;
    int row_div;
    float* row_sq;
    float* col_part;
    const float* row_sub;
    const float* A1;
    const float* A2;
    const float* B1;
    const float* B2;
    int k_seg;
};
static_assert(sizeof(GemmArgs) == 216, "kernel argument layout of forge::GemmArgs");

// Must match forge::GemmBatchArgs in csrc/kernels/gemm.hpp.
constexpr int GEMM_BATCH_MAX = 8;
struct GemmBatchArgs {
    GemmArgs p[GEMM_BATCH_MAX];
    int count;
    int tiles;
};

// Must match forge::RowArgs in csrc/kernels/rows.hpp.
struct RowArgs {
    const float* x;
    float* y;
    const float* dy;
    const float* gamma;
    const float* beta;
    float* pgamma;
    float* pbeta;
    int rows, cols;
    float eps;
    float scale;
    int nt_stores = 0;   // set by row_launch
    int lds_params = 0;  // set by row_launch
    const float* dsub = nullptr;  // norm backward row dot
    float* dot = nullptr;
    float dscale = 1.0f;
};

// LayerNorm forward stages gamma/beta in LDS below this many elements
// (rows.hpp; the same 64 MiB as STREAM_NT_MIN in common.hpp).
constexpr long long kRowLdsParamsMax = 16ll << 20;

// Must match forge::ColSumOut in csrc/kernels/elementwise.hpp: where a final
// column-sum pass writes (out, when not null) and the parameter vector whose
// SGD step it applies (param -= lr * sum, when not null).
struct ColSumOut {
    float* out;
    float* param;
    float lr;
};

constexpr int ROW_WAVES = 4;   // rows.hpp ROW_WAVES
constexpr int ROW_PARTIAL_WAVES = 8;  // rows.hpp ROW_PARTIAL_WAVES
constexpr int EW_THREADS = 256;  // elementwise.hpp EW_THREADS

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

}  // namespace

// Per-stream scratch for multi-pass kernels (column partials, reduction
// partials).  Each stream owns one so concurrent streams never share it.
struct Workspace {
    float* ptr = nullptr;
    size_t len = 0;
};

struct forge_stream {
    hipStream_t stream = nullptr;
    hipEvent_t event = nullptr;
    Workspace ws;
};

struct forge_runtime {
    int device = 0;
    forge_stream primary;
    hipModule_t module = nullptr;
    std::unordered_map<std::string, hipFunction_t> functions;
    std::unordered_map<std::string, int> occupancy;  // GEMM kernels: workgroups per CU
    std::unordered_map<size_t, std::vector<float*>> pool;
    std::vector<forge_stream*> streams;
    int cu_count = 0;
    size_t lds_bytes = 0;
    int clock_khz = 0;
    char arch[256] = {0};
    // Device address of this device's no-allocation scratch array
    // (noalloc_scratch.hip), resolved at creation; null if that failed.
    float* noalloc_scratch = nullptr;
    hipError_t noalloc_status = hipSuccess;
};

namespace {

forge_stream* pick(forge_runtime* rt, forge_stream* s) { return s ? s : &rt->primary; }

forge_status get_function(forge_runtime* rt, const char* name, hipFunction_t* out) {
    auto it = rt->functions.find(name);
    if (it != rt->functions.end()) {
        *out = it->second;
        return FORGE_OK;
    }
    hipFunction_t f = nullptr;
    hipError_t e = hipModuleGetFunction(&f, rt->module, name);
    if (e != hipSuccess)
        return fail(FORGE_ENOMODULE, "kernel %s not found in code object: %s", name,
                    hipGetErrorString(e));
    rt->functions.emplace(name, f);
    *out = f;
    return FORGE_OK;
}

// Launches `name` with the given argument addresses (kernelParams form).
forge_status launch(forge_runtime* rt, forge_stream* s, const char* name, dim3 grid,
                    dim3 block, size_t shmem, void** args) {
    if (grid.x == 0 || grid.y == 0 || grid.z == 0) return FORGE_OK;
    hipFunction_t f;
    FORGE_TRY(get_function(rt, name, &f));
    HIP_TRY(hipModuleLaunchKernel(f, grid.x, grid.y, grid.z, block.x, block.y, block.z,
                                  (unsigned)shmem, pick(rt, s)->stream, args, nullptr));
    return FORGE_OK;
}

template <typename... T>
forge_status launch_args(forge_runtime* rt, forge_stream* s, const char* name, dim3 grid,
                         dim3 block, size_t shmem, T... values) {
    void* args[] = {static_cast<void*>(&values)...};
    return launch(rt, s, name, grid, block, shmem, args);
}

forge_status workspace(forge_runtime* rt, forge_stream* s, size_t n, float** out) {
    forge_stream* st = pick(rt, s);
    if (st->ws.len < n) {
        if (st->ws.ptr) {
            // Work queued on this stream may still read the old buffer.
            HIP_TRY(hipStreamSynchronize(st->stream));
            HIP_TRY(hipFree(st->ws.ptr));
            st->ws = Workspace{};
        }
        size_t len = std::max<size_t>(n, 1 << 20);
        void* p = nullptr;
        if (hipMalloc(&p, len * sizeof(float)) != hipSuccess)
            return fail(FORGE_ENOMEM, "workspace allocation of %zu floats failed", len);
        st->ws.ptr = static_cast<float*>(p);
        st->ws.len = len;
    }
    *out = st->ws.ptr;
    return FORGE_OK;
}

forge_status need(const forge_slice& s, size_t n, const char* what) {
    if (n > 0 && (s.ptr == nullptr || s.len < n))
        return fail(FORGE_EINVAL, "%s: slice of %zu elements (ptr %p) is too short for %zu",
                    what, s.len, (void*)s.ptr, n);
    return FORGE_OK;
}

forge_status need(const forge_slice_u32& s, size_t n, const char* what) {
    if (n > 0 && (s.ptr == nullptr || s.len < n))
        return fail(FORGE_EINVAL, "%s: u32 slice of %zu elements (ptr %p) is too short for %zu",
                    what, s.len, (void*)s.ptr, n);
    return FORGE_OK;
}

forge_status need_opt(const forge_slice& s, size_t n, const char* what) {
    if (s.ptr == nullptr) return FORGE_OK;
    return need(s, n, what);
}

bool fits_int(size_t v) { return v <= 0x7fffffffu; }

unsigned grid_for(long long work_items, long long per_block, unsigned cap) {
    long long g = (work_items + per_block - 1) / per_block;
    if (g < 1) g = 1;
    if (g > cap) g = cap;
    return (unsigned)g;
}

// Grid of the vectorised streaming kernels (elementwise.hpp stream_f4) for
// n4 float4 items: one item per thread.
unsigned stream_grid(long long n4) { return grid_for(n4, EW_THREADS, 1u << 30); }

std::string default_module_path() {
    if (const char* env = getenv("OXFORGE_KERNELS")) return env;
    Dl_info info;
    if (dladdr(reinterpret_cast<void*>(&forge_runtime_create), &info) && info.dli_fname) {
        std::string p(info.dli_fname);
        size_t slash = p.rfind('/');
        std::string dir = slash == std::string::npos ? "." : p.substr(0, slash);
        return dir + "/oxforge_kernels.hsaco";
    }
    return "oxforge_kernels.hsaco";
}

}  // namespace

// ================================================================ lifecycle

extern "C" forge_status forge_device_count(int* count) {
    if (!count) return fail(FORGE_EINVAL, "count is null");
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) n = 0;
    *count = n;
    return FORGE_OK;
}

extern "C" const char* forge_status_string(forge_status s) {
    switch (s) {
    case FORGE_OK: return "ok";
    case FORGE_EINVAL: return "invalid argument";
    case FORGE_ENOMEM: return "out of memory";
    case FORGE_EHIP: return "HIP runtime error";
    case FORGE_ENOMODULE: return "code object or kernel missing";
    case FORGE_ENODEV: return "no HIP device";
    case FORGE_EIO: return "file I/O failed";
    }
    return "unknown status";
}

extern "C" const char* forge_last_error(void) { return g_last_error.c_str(); }

// Lets the executor entry points (net_capi.cpp) report exceptions through
// forge_last_error(); not part of the public ABI.
extern "C" void forge_internal_set_error(const char* message) {
    g_last_error = message ? message : "";
}

extern "C" forge_status forge_runtime_create(int device, const char* module_path,
                                             forge_runtime** out) {
    if (!out) return fail(FORGE_EINVAL, "out is null");
    *out = nullptr;
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess || n == 0)
        return fail(FORGE_ENODEV, "no HIP device is visible");
    if (device < 0 || device >= n)
        return fail(FORGE_ENODEV, "device %d requested, %d visible", device, n);
    std::string path = module_path ? module_path : default_module_path();
    FILE* f = fopen(path.c_str(), "rb");
    if (!f) return fail(FORGE_ENOMODULE, "code object %s not found", path.c_str());
    fclose(f);

    HIP_TRY(hipSetDevice(device));
    auto* rt = new forge_runtime();
    rt->device = device;
    hipError_t e = hipModuleLoad(&rt->module, path.c_str());
    if (e != hipSuccess) {
        delete rt;
        return fail(FORGE_ENOMODULE, "hipModuleLoad(%s): %s", path.c_str(), hipGetErrorString(e));
    }
    if (hipStreamCreateWithFlags(&rt->primary.stream, hipStreamNonBlocking) != hipSuccess ||
        hipEventCreateWithFlags(&rt->primary.event, hipEventDisableTiming) != hipSuccess) {
        (void)hipModuleUnload(rt->module);
        delete rt;
        return fail(FORGE_EHIP, "primary stream creation failed");
    }
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, device) == hipSuccess) {
        rt->cu_count = prop.multiProcessorCount;
        rt->lds_bytes = prop.sharedMemPerBlock;
        rt->clock_khz = prop.clockRate;
        snprintf(rt->arch, sizeof rt->arch, "%s", prop.gcnArchName);
    }
    // Once per runtime, with the device current: the address of the device's
    // copy of the no-allocation scratch array.  A failure here disables only
    // forge_layer_norm_bwd_noalloc, which then reports it.
    rt->noalloc_status = forge_internal_noalloc_scratch(&rt->noalloc_scratch);
    *out = rt;
    return FORGE_OK;
}

extern "C" forge_status forge_runtime_destroy(forge_runtime* rt) {
    if (!rt) return FORGE_OK;
    (void)hipSetDevice(rt->device);
    (void)hipDeviceSynchronize();
    for (auto& kv : rt->pool)
        for (float* p : kv.second) (void)hipFree(p);
    for (forge_stream* s : rt->streams) {
        if (s->ws.ptr) (void)hipFree(s->ws.ptr);
        (void)hipEventDestroy(s->event);
        (void)hipStreamDestroy(s->stream);
        delete s;
    }
    if (rt->primary.ws.ptr) (void)hipFree(rt->primary.ws.ptr);
    (void)hipEventDestroy(rt->primary.event);
    (void)hipStreamDestroy(rt->primary.stream);
    (void)hipModuleUnload(rt->module);
    delete rt;
    return FORGE_OK;
}

extern "C" forge_status forge_sync(forge_runtime* rt, forge_stream* s) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    HIP_TRY(hipStreamSynchronize(pick(rt, s)->stream));
    return FORGE_OK;
}

extern "C" forge_status forge_device_props(forge_runtime* rt, int* cu_count, size_t* lds_bytes,
                                           int* clock_khz, char* arch, size_t arch_len) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (cu_count) *cu_count = rt->cu_count;
    if (lds_bytes) *lds_bytes = rt->lds_bytes;
    if (clock_khz) *clock_khz = rt->clock_khz;
    if (arch && arch_len) snprintf(arch, arch_len, "%s", rt->arch);
    return FORGE_OK;
}

// ================================================================== streams

extern "C" forge_status forge_streams_create(forge_runtime* rt, size_t n, forge_stream** out) {
    if (!rt || (n && !out)) return fail(FORGE_EINVAL, "null argument");
    HIP_TRY(hipEventRecord(rt->primary.event, rt->primary.stream));
    for (size_t i = 0; i < n; i++) {
        auto* s = new forge_stream();
        if (hipStreamCreateWithFlags(&s->stream, hipStreamNonBlocking) != hipSuccess ||
            hipEventCreateWithFlags(&s->event, hipEventDisableTiming) != hipSuccess) {
            if (s->event) (void)hipEventDestroy(s->event);
            if (s->stream) (void)hipStreamDestroy(s->stream);
            delete s;
            return fail(FORGE_EHIP, "stream creation failed");
        }
        // CudaStream::fork: the new stream starts after the primary's work.
        HIP_TRY(hipStreamWaitEvent(s->stream, rt->primary.event, 0));
        rt->streams.push_back(s);
        out[i] = s;
    }
    return FORGE_OK;
}

extern "C" forge_status forge_streams_fork(forge_runtime* rt, size_t n,
                                           forge_stream* const* streams) {
    if (!rt || (n && !streams)) return fail(FORGE_EINVAL, "null argument");
    HIP_TRY(hipEventRecord(rt->primary.event, rt->primary.stream));
    for (size_t i = 0; i < n; i++)
        HIP_TRY(hipStreamWaitEvent(streams[i]->stream, rt->primary.event, 0));
    return FORGE_OK;
}

extern "C" forge_status forge_streams_join(forge_runtime* rt, size_t n,
                                           forge_stream* const* streams) {
    if (!rt || (n && !streams)) return fail(FORGE_EINVAL, "null argument");
    for (size_t i = 0; i < n; i++) {
        HIP_TRY(hipEventRecord(streams[i]->event, streams[i]->stream));
        HIP_TRY(hipStreamWaitEvent(rt->primary.stream, streams[i]->event, 0));
    }
    return FORGE_OK;
}

extern "C" forge_status forge_stream_wait(forge_runtime* rt, forge_stream* waiter,
                                          forge_stream* signaler) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    forge_stream* w = pick(rt, waiter);
    forge_stream* g = pick(rt, signaler);
    if (w == g) return FORGE_OK;
    HIP_TRY(hipEventRecord(g->event, g->stream));
    HIP_TRY(hipStreamWaitEvent(w->stream, g->event, 0));
    return FORGE_OK;
}

extern "C" forge_status forge_stream_destroy(forge_runtime* rt, forge_stream* s) {
    if (!rt || !s) return fail(FORGE_EINVAL, "null argument");
    auto it = std::find(rt->streams.begin(), rt->streams.end(), s);
    if (it == rt->streams.end()) return fail(FORGE_EINVAL, "stream not owned by this runtime");
    HIP_TRY(hipStreamSynchronize(s->stream));
    if (s->ws.ptr) (void)hipFree(s->ws.ptr);
    (void)hipEventDestroy(s->event);
    (void)hipStreamDestroy(s->stream);
    rt->streams.erase(it);
    delete s;
    return FORGE_OK;
}

extern "C" forge_status forge_stream_workspace_floats(forge_runtime* rt, forge_stream* s,
                                                      size_t* floats) {
    if (!rt || !floats) return fail(FORGE_EINVAL, "null argument");
    if (s && std::find(rt->streams.begin(), rt->streams.end(), s) == rt->streams.end())
        return fail(FORGE_EINVAL, "stream not owned by this runtime");
    *floats = pick(rt, s)->ws.len;
    return FORGE_OK;
}

// =================================================================== events

struct forge_event {
    hipEvent_t event = nullptr;
};

extern "C" forge_status forge_event_create(forge_runtime* rt, forge_event** out) {
    if (!rt || !out) return fail(FORGE_EINVAL, "null argument");
    auto* e = new forge_event();
    if (hipEventCreate(&e->event) != hipSuccess) {
        delete e;
        return fail(FORGE_EHIP, "hipEventCreate failed");
    }
    *out = e;
    return FORGE_OK;
}

extern "C" forge_status forge_event_record(forge_runtime* rt, forge_stream* s, forge_event* ev) {
    if (!rt || !ev) return fail(FORGE_EINVAL, "null argument");
    HIP_TRY(hipEventRecord(ev->event, pick(rt, s)->stream));
    return FORGE_OK;
}

extern "C" forge_status forge_event_elapsed_ms(forge_runtime* rt, forge_event* start,
                                               forge_event* end, float* ms) {
    if (!rt || !start || !end || !ms) return fail(FORGE_EINVAL, "null argument");
    HIP_TRY(hipEventSynchronize(end->event));
    HIP_TRY(hipEventElapsedTime(ms, start->event, end->event));
    return FORGE_OK;
}

extern "C" forge_status forge_event_destroy(forge_runtime* rt, forge_event* ev) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (!ev) return FORGE_OK;
    (void)hipEventDestroy(ev->event);
    delete ev;
    return FORGE_OK;
}

// =================================================================== memory

extern "C" forge_status forge_alloc(forge_runtime* rt, size_t n, forge_slice* out) {
    if (!rt || !out) return fail(FORGE_EINVAL, "null argument");
    out->ptr = nullptr;
    out->len = 0;
    if (n == 0) return FORGE_OK;
    auto it = rt->pool.find(n);
    if (it != rt->pool.end() && !it->second.empty()) {
        out->ptr = it->second.back();
        it->second.pop_back();
        out->len = n;
        return FORGE_OK;
    }
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, n * sizeof(float));
    if (e != hipSuccess)
        return fail(FORGE_ENOMEM, "hipMalloc of %zu floats: %s", n, hipGetErrorString(e));
    out->ptr = static_cast<float*>(p);
    out->len = n;
    return FORGE_OK;
}

extern "C" forge_status forge_alloc_zeroed(forge_runtime* rt, size_t n, forge_slice* out) {
    FORGE_TRY(forge_alloc(rt, n, out));
    return forge_fill(rt, nullptr, *out, 0.0f);
}

extern "C" forge_status forge_recycle(forge_runtime* rt, forge_slice buf) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (!buf.ptr || buf.len == 0) return FORGE_OK;
    rt->pool[buf.len].push_back(buf.ptr);
    return FORGE_OK;
}

extern "C" forge_status forge_free(forge_runtime* rt, forge_slice buf) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (!buf.ptr) return FORGE_OK;
    HIP_TRY(hipStreamSynchronize(rt->primary.stream));
    HIP_TRY(hipFree(buf.ptr));
    return FORGE_OK;
}

extern "C" forge_status forge_alloc_u32(forge_runtime* rt, size_t n, forge_slice_u32* out) {
    if (!rt || !out) return fail(FORGE_EINVAL, "null argument");
    out->ptr = nullptr;
    out->len = 0;
    if (n == 0) return FORGE_OK;
    void* p = nullptr;
    hipError_t e = hipMalloc(&p, n * sizeof(uint32_t));
    if (e != hipSuccess)
        return fail(FORGE_ENOMEM, "hipMalloc of %zu u32: %s", n, hipGetErrorString(e));
    out->ptr = static_cast<uint32_t*>(p);
    out->len = n;
    return FORGE_OK;
}

extern "C" forge_status forge_free_u32(forge_runtime* rt, forge_slice_u32 buf) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (!buf.ptr) return FORGE_OK;
    HIP_TRY(hipStreamSynchronize(rt->primary.stream));
    HIP_TRY(hipFree(buf.ptr));
    return FORGE_OK;
}

extern "C" forge_status forge_reserve(forge_runtime* rt, size_t n, size_t count) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (n == 0) return FORGE_OK;
    auto& v = rt->pool[n];
    while (v.size() < count) {
        void* p = nullptr;
        hipError_t e = hipMalloc(&p, n * sizeof(float));
        if (e != hipSuccess)
            return fail(FORGE_ENOMEM, "hipMalloc of %zu floats: %s", n, hipGetErrorString(e));
        v.push_back(static_cast<float*>(p));
    }
    return FORGE_OK;
}

extern "C" forge_status forge_pool_count(forge_runtime* rt, size_t n, size_t* count) {
    if (!rt || !count) return fail(FORGE_EINVAL, "null argument");
    auto it = rt->pool.find(n);
    *count = it == rt->pool.end() ? 0 : it->second.size();
    return FORGE_OK;
}

extern "C" forge_status forge_memcpy_h2d(forge_runtime* rt, forge_slice dst, const float* src,
                                         size_t n) {
    if (!rt || (n && !src)) return fail(FORGE_EINVAL, "null argument");
    FORGE_TRY(need(dst, n, "memcpy_h2d dst"));
    if (n == 0) return FORGE_OK;
    HIP_TRY(hipMemcpyAsync(dst.ptr, src, n * sizeof(float), hipMemcpyHostToDevice,
                           rt->primary.stream));
    HIP_TRY(hipStreamSynchronize(rt->primary.stream));
    return FORGE_OK;
}

extern "C" forge_status forge_memcpy_d2h(forge_runtime* rt, float* dst, forge_slice src,
                                         size_t n) {
    if (!rt || (n && !dst)) return fail(FORGE_EINVAL, "null argument");
    FORGE_TRY(need(src, n, "memcpy_d2h src"));
    if (n == 0) return FORGE_OK;
    HIP_TRY(hipMemcpyAsync(dst, src.ptr, n * sizeof(float), hipMemcpyDeviceToHost,
                           rt->primary.stream));
    HIP_TRY(hipStreamSynchronize(rt->primary.stream));
    return FORGE_OK;
}

extern "C" forge_status forge_memcpy_d2h_u32(forge_runtime* rt, uint32_t* dst, forge_slice_u32 src,
                                             size_t n) {
    if (!rt || (n && !dst)) return fail(FORGE_EINVAL, "null argument");
    FORGE_TRY(need(src, n, "memcpy_d2h_u32 src"));
    if (n == 0) return FORGE_OK;
    HIP_TRY(hipMemcpyAsync(dst, src.ptr, n * sizeof(uint32_t), hipMemcpyDeviceToHost,
                           rt->primary.stream));
    HIP_TRY(hipStreamSynchronize(rt->primary.stream));
    return FORGE_OK;
}

extern "C" forge_status forge_memcpy_d2d(forge_runtime* rt, forge_stream* s, forge_slice dst,
                                         forge_slice src, size_t n) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(need(dst, n, "memcpy_d2d dst"));
    FORGE_TRY(need(src, n, "memcpy_d2d src"));
    if (n == 0) return FORGE_OK;
    HIP_TRY(hipMemcpyAsync(dst.ptr, src.ptr, n * sizeof(float), hipMemcpyDeviceToDevice,
                           pick(rt, s)->stream));
    return FORGE_OK;
}

extern "C" forge_status forge_fill(forge_runtime* rt, forge_stream* s, forge_slice x, float value) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (!x.ptr || x.len == 0) return FORGE_OK;
    long long n = (long long)x.len;
    bool vec = aligned16(x.ptr);
    unsigned g = vec ? stream_grid(n / 4 + 1) : grid_for(n, EW_THREADS, 8192);
    return launch_args(rt, s, vec ? "forge_fill_v" : "forge_fill_s", dim3(g), dim3(EW_THREADS), 0,
                       x.ptr, n, value);
}

// ================================================================== kernels

namespace {

struct GemmConfig {
    const char* tag;  // e.g. "128x128x32_x"
    int bm, bn, bk, threads;
};

const char* gemm_ab(int ta, int tb) {
    static const char ab[2][2][3] = {{"nn", "nt"}, {"tn", "tt"}};
    return ab[ta ? 1 : 0][tb ? 1 : 0];
}

const GemmConfig kTile128x256 = {"128x256x32_x", 128, 256, 32, 256};
const GemmConfig kTile128x128 = {"128x128x32_x", 128, 128, 32, 256};
const GemmConfig kTile128x64 = {"128x64x32_x", 128, 64, 32, 256};
const GemmConfig kTile64x128 = {"64x128x32_x", 64, 128, 32, 256};
const GemmConfig kTile64x64 = {"64x64x32_x", 64, 64, 32, 256};
const GemmConfig kTile64x128w8 = {"64x128x32_x8", 64, 128, 32, 512};
const GemmConfig kGuard64 = {"64x64x16_2x2_g", 64, 64, 16, 256};

// Unguarded tiles, largest first, and their measured efficiency relative to
// 128x128 on large shapes with every CU holding two or more workgroups
// (MI355X, e.g. 4096x4096x2048 plain: 148.9, 146.0, 145.4 and 138.3
// TFLOP/s for 128x128, 64x128 and 128x64 at two per CU, and 64x64).  All
// but 128x256 have fused-epilogue and batched instances; 128x256 has a
// plain NN one.
// The eight-wave 64x128 tile (two waves per SIMD) serves plain products
// (forge_gemm_f32): 4096^3 at 150.2-150.7 TFLOP/s against 149.6-149.8 for
// 128x128 on one device, 8192x1024x4096 at 150.0 against 148.5.  Fused
// products keep the four-wave tiles: although the eight-wave tile also ran
// faster on most C4/C5 NN and NT products in isolation (2048x1024x4096 with
// bias 143.9 against 141.6), the C4 forward was no faster with it (0.521 ms
// both ways) and the C5 step 0.5% slower (11.54 against 11.48 ms); batched
// Q/K/V lost 7% (98.3 against 92.0 us at C4), and TN products, whose
// transposed A it reads 32 bits at a time (16-row wave sub-tiles), lost
// 0.3-1%.  Measured again with the fused NN and NT products (not TN, not
// the K-segmented one) on the eight-wave tile, in ABBA pairs on one box:
// C4 0.5393-0.5397 against 0.5165-0.5191 ms, C5 11.266-11.301 against
// 11.224-11.287 ms.
const GemmConfig* const kUnguarded[] = {&kTile128x256, &kTile128x128, &kTile128x64,
                                        &kTile64x128, &kTile64x64, &kTile64x128w8};
// From K = 2048 on, 128x128 scores below 64x128 (tile_efficiency), so
// longer products whose tiles balance either way take 64x128: in the C5
// step (K 2048-8192) that measured 11,243 against 11,272 us by kernel trace
// on one box (two traces each; six of the nine products with K >= 4096
// gained 2-8 us, the two 4096x8192x2048 products lost 3-7 us) and 11.220
// against 11.255 ms in six ABBA pairs of bench runs, each pair faster.  Up to K = 1024 128x128 keeps 1.0:
// the C4 FFN up-projection (K 1024) as 64x128 made the C4 forward about
// 0.5 us slower in three of four pairs.  Two variants measured within the
// noise of eight pairs each: 128x128 at 1.0 up to K = 2048 (C5 -7 us), and
// the batched C5 products held to two workgroups per CU (-6 us).
const double kTileEfficiency[] = {0.975, 0.98, 0.98, 0.985, 0.94, 1.005};
constexpr int kUnguardedCount = 6;
// A CU that holds a single four-wave workgroup has one wave per SIMD, which
// hides less: 2048x2048x1024 as 256 tiles of 128x128 runs at 133 TFLOP/s,
// as 512 tiles of 64x128 at 139.
constexpr double kSingleWorkgroupFactor = 0.96;

enum class GemmKind { Plain, Epilogue, Batch, Stats, RowSub, SegK };

// Kernel that runs a tile: plain NN (forge_gemm_nn_<tile>), fused epilogue
// (forge_gemm_<ab>_<tile>_e), fused epilogue with row statistics and column
// sums (forge_gemm_<ab>_<tile>_s), the same with the row subtrahend
// (forge_gemm_<ab>_<tile>_r), fused epilogue over K segments
// (forge_gemm_<ab>_<tile>_k) or batched (forge_gemm_batch_<ab>_<tile>).
void gemm_kernel_name(char* out, size_t cap, GemmKind kind, int ta, int tb,
                      const GemmConfig& cfg) {
    if (kind == GemmKind::Batch)
        snprintf(out, cap, "forge_gemm_batch_%s_%s", gemm_ab(ta, tb), cfg.tag);
    else
        snprintf(out, cap, "forge_gemm_%s_%s%s", gemm_ab(ta, tb), cfg.tag,
                 kind == GemmKind::Epilogue ? "_e"
                 : kind == GemmKind::Stats  ? "_s"
                 : kind == GemmKind::RowSub ? "_r"
                 : kind == GemmKind::SegK   ? "_k"
                                            : "");
}

// Workgroups of a kernel that one CU holds at once (its registers and LDS),
// from the loaded code object; cached per kernel.
int gemm_occupancy(forge_runtime* rt, const char* name, int threads) {
    auto it = rt->occupancy.find(name);
    if (it != rt->occupancy.end()) return it->second;
    int blocks = 1;
    hipFunction_t f = nullptr;
    if (get_function(rt, name, &f) == FORGE_OK &&
        hipModuleOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, f, threads, 0) != hipSuccess)
        blocks = 1;
    blocks = blocks < 1 ? 1 : blocks;
    rt->occupancy.emplace(name, blocks);
    return blocks;
}

// Dynamic LDS that limits a kernel to `cap` resident workgroups per CU (its
// static LDS plus this fills 1 / cap of the CU's LDS); 0 when the kernel's
// own LDS already allows no more.
forge_status occupancy_cap_shmem(forge_runtime* rt, const char* name, int cap, size_t* out) {
    hipFunction_t f = nullptr;
    FORGE_TRY(get_function(rt, name, &f));
    int static_lds = 0, lds_cu = 0;
    HIP_TRY(hipFuncGetAttribute(&static_lds, HIP_FUNC_ATTRIBUTE_SHARED_SIZE_BYTES, f));
    HIP_TRY(hipDeviceGetAttribute(&lds_cu, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
                                  rt->device));
    const int total = (lds_cu / cap) & ~511;
    *out = total > static_lds ? (size_t)(total - static_lds) : 0;
    return FORGE_OK;
}

// A tile and how many of its workgroups a CU may hold (cap 0: as many as
// its registers and LDS allow; otherwise the launch reserves extra LDS).
struct GemmPlan {
    const GemmConfig* cfg;
    int cap;
};

// Tile i's factor for a product of depth K: kTileEfficiency (128x128 at
// 1.0 up to K = 1024), or the comma-separated factors of $OXFORGE_GEMM_EFF
// in the order of kUnguarded (a tuning knob).
double tile_efficiency(int i, size_t K) {
    static const std::vector<double> env = [] {
        std::vector<double> v;
        if (const char* e = getenv("OXFORGE_GEMM_EFF")) {
            char* end = nullptr;
            for (const char* p = e; *p; p = *end ? end + 1 : end) {
                v.push_back(strtod(p, &end));
                if (end == p) break;
            }
        }
        return v;
    }();
    if ((size_t)i < env.size()) return env[(size_t)i];
    if (kUnguarded[i] == &kTile128x128 && K <= 1024) return 1.0;
    return kTileEfficiency[i];
}

// Tile choice: the best efficiency x balance over the tiles and, for each,
// the number c of workgroups a CU may hold (from what fits down to one).
// t tiles that all fit at once (t <= CUs * c) spread over the CUs, balance
// t / (CUs * ceil(t / CUs)); more than that run in waves of CUs * c,
// balance t / (CUs * c * ceil(t / (CUs * c))).  The last of a wave's tiles
// do not spread evenly over the CUs: 1024 tiles of 64x128 at three per CU
// run at 120 TFLOP/s, at two per CU (exact waves) at 147.  A CU left with
// a single four-wave workgroup scores kSingleWorkgroupFactor less (an
// eight-wave one does not: it has two waves per SIMD).  Ties go to the
// larger tile, then to the larger c.  Results on the C3-C5 shapes: plain
// 4096^3 and 8192x1024x4096 -> the eight-wave 64x128; the C4 FFN
// up-projection -> 128x128; the other fused and batched C4 and C5 products
// -> 64x128 (the three C4 Q/K/V products of one batch: 768 tiles at three
// per CU).  Unaligned shapes and shapes the tiles do not
// divide take the bounds-guarded 64x64 tile.  `count` same-shape products
// share the launch (kind Batch).
GemmPlan choose_gemm(forge_runtime* rt, int ta, int tb, size_t M, size_t N, size_t K,
                     bool aligned, GemmKind kind, size_t count = 1) {
    const size_t cus = rt->cu_count > 0 ? (size_t)rt->cu_count : 256;
    GemmPlan best{&kGuard64, 0};
    double best_score = 0.0;
    const bool plain_nn = kind == GemmKind::Plain && !ta && !tb;
    for (int i = plain_nn ? 0 : 1; i < kUnguardedCount; i++) {
        const GemmConfig& g = *kUnguarded[i];
        if (!aligned || M % g.bm || N % g.bn || K % (size_t)g.bk) continue;
        if (&g == &kTile64x128w8 && kind != GemmKind::Plain) continue;
        char name[96];
        gemm_kernel_name(name, sizeof name, kind, ta, tb, g);
        const int occ = gemm_occupancy(rt, name, g.threads);
        const size_t t = count * (M / g.bm) * (N / g.bn);
        for (int c = occ; c >= 1; c--) {
            const size_t slots = cus * (size_t)c;
            const size_t per_cu = (t + cus - 1) / cus;
            const double balance =
                t <= slots ? (double)t / (double)(cus * per_cu)
                           : (double)t / (double)(slots * ((t + slots - 1) / slots));
            // (an eight-wave workgroup alone on a CU still has two waves per SIMD)
            const bool single = g.threads == 256 && occ > 1 && (c == 1 || per_cu == 1);
            const double score =
                tile_efficiency(i, K) * balance * (single ? kSingleWorkgroupFactor : 1.0);
            if (score > best_score + 1e-9) {
                best = {&g, c == occ ? 0 : c};
                best_score = score;
            }
        }
    }
    return best;
}

// Split-K plan for one product.  With the four-wave tiles no C3/C4/C5 shape
// gains from a split (bench.py --sweep: e.g. 2048x1024x4096 122.5 TFLOP/s
// unsplit against 117.5 in four slices), so products are split only when
// the chosen tile leaves at least three quarters of the CUs idle: the K
// slices are doubled while the launch still fits on the CUs and each slice
// keeps >= 1024 of K (up to eight).  Returns the split count and sets *cfg
// to the tile to use.
int choose_splits(forge_runtime* rt, int ta, int tb, size_t M, size_t N, size_t K, bool aligned,
                  const GemmConfig** cfg) {
    const size_t cus = rt->cu_count > 0 ? (size_t)rt->cu_count : 256;
    // The K slices run as one batched launch.
    const GemmConfig& g = *choose_gemm(rt, ta, tb, M, N, K, aligned, GemmKind::Batch).cfg;
    if (&g == &kGuard64) return 1;
    const size_t t = (M / g.bm) * (N / g.bn);
    if (t * 4 > cus) return 1;
    int splits = 1;
    while (splits * 2 <= GEMM_BATCH_MAX && t * (size_t)splits * 2 <= cus &&
           K % ((size_t)splits * 2 * g.bk) == 0 && K / ((size_t)splits * 2) >= 1024)
        splits *= 2;
    if (splits > 1) *cfg = &g;
    return splits;
}

constexpr long long kUnguardedMaxPitch = 1LL << 21;

// Validates one product and fills its kernel arguments; *aligned reports
// whether the unguarded tiles may read the operands.
forge_status gemm_args(int ta, int tb, forge_slice A, forge_slice B, forge_slice C, size_t M,
                       size_t N, size_t K, const forge_gemm_epilogue* ep, GemmArgs* out,
                       bool* aligned) {
    if (!fits_int(M) || !fits_int(N) || !fits_int(K))
        return fail(FORGE_EINVAL, "gemm dimensions exceed 2^31-1");
    FORGE_TRY(need(A, M * K, "gemm A"));
    FORGE_TRY(need(B, K * N, "gemm B"));
    FORGE_TRY(need(C, M * N, "gemm C"));
    GemmArgs a{};
    a.A = A.ptr;
    a.B = B.ptr;
    a.C = C.ptr;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.lda = ta ? (long long)M : (long long)K;
    a.ldb = tb ? (long long)K : (long long)N;
    a.ldc = (long long)N;
    a.alpha = 1.0f;
    // The unguarded tiles also keep their slab offsets (up to 256 rows of
    // an operand) below 2^31 bytes: row pitches up to 2^21 floats.
    bool al = aligned16(A.ptr) && aligned16(B.ptr) && aligned16(C.ptr) && a.lda % 4 == 0 &&
              a.ldb % 4 == 0 && a.lda <= kUnguardedMaxPitch && a.ldb <= kUnguardedMaxPitch;
    if (ep) {
        FORGE_TRY(need_opt(ep->bias, N, "gemm bias"));
        FORGE_TRY(need_opt(ep->residual, M * N, "gemm residual"));
        FORGE_TRY(need_opt(ep->aux_mul, M * N, "gemm aux_mul"));
        FORGE_TRY(need_opt(ep->pre_out, M * N, "gemm pre_out"));
        if (ep->activation < FORGE_ACT_IDENTITY || ep->activation > FORGE_ACT_SILU)
            return fail(FORGE_EINVAL, "unknown activation %d", ep->activation);
        if (ep->aux_activation < FORGE_ACT_IDENTITY || ep->aux_activation > FORGE_ACT_SILU)
            return fail(FORGE_EINVAL, "unknown aux activation %d", ep->aux_activation);
        // The unguarded tiles move epilogue operands as 128-bit accesses.
        for (const forge_slice* e : {&ep->bias, &ep->residual, &ep->aux_mul, &ep->pre_out})
            if (e->ptr && !aligned16(e->ptr)) al = false;
        a.alpha = ep->alpha;
        a.bias = ep->bias.ptr;
        a.residual = ep->residual.ptr;
        a.aux = ep->aux_mul.ptr;
        a.pre_out = ep->pre_out.ptr;
        a.act = ep->activation;
        a.aux_act = ep->aux_activation;
        a.update = ep->update ? 1 : 0;
        a.update_scale = ep->update_scale;
        if (ep->row_parts_in.ptr) {
            if (ep->row_parts == 0 || ep->row_n == 0)
                return fail(FORGE_EINVAL, "gemm row statistics need row_parts and row_n >= 1");
            if (ep->row_div < 0 || ep->row_div > 3)
                return fail(FORGE_EINVAL, "gemm row_div %d is not 0-3", ep->row_div);
            if (!fits_int(ep->row_parts) || !fits_int(ep->row_n))
                return fail(FORGE_EINVAL, "gemm row_parts / row_n exceed 2^31-1");
            FORGE_TRY(need(ep->row_parts_in, M * ep->row_parts, "gemm row_parts_in"));
            a.row_part = ep->row_parts_in.ptr;
            a.row_parts = (int)ep->row_parts;
            a.row_n = (int)ep->row_n;
            a.row_eps = ep->row_eps;
            a.row_div = ep->row_div;
        } else if (ep->row_div) {
            return fail(FORGE_EINVAL, "gemm row_div without row_parts_in");
        }
        FORGE_TRY(need_opt(ep->row_sumsq_out, M * ((N + 31) / 32), "gemm row_sumsq_out"));
        FORGE_TRY(need_opt(ep->col_sums_out, N, "gemm col_sums_out"));
        FORGE_TRY(need_opt(ep->col_sums_param, N, "gemm col_sums_param"));
        FORGE_TRY(need_opt(ep->row_sub, M, "gemm row_sub"));
        a.row_sq = ep->row_sumsq_out.ptr;
        a.row_sub = ep->row_sub.ptr;
    }
    *out = a;
    *aligned = al;
    return FORGE_OK;
}

// Epilogues that need the statistics instances on the unguarded tiles (_s,
// or _r with the row subtrahend): row statistics, column sums, row_sub.  The
// plain fused instances (_e) carry none of that code.
bool gemm_has_stats(const forge_gemm_epilogue* ep) {
    return ep && (ep->row_parts_in.ptr || ep->row_sumsq_out.ptr || ep->col_sums_out.ptr ||
                  ep->col_sums_param.ptr || ep->row_sub.ptr);
}

// Split-K: `splits` K slices of the product as one batched launch writing
// raw partial products to the stream's workspace, then one kernel summing
// them in slice order and applying a's epilogue.  Requires an unguarded
// tile and K % (splits * bk) == 0.
forge_status gemm_split_launch(forge_runtime* rt, forge_stream* s, int ta, int tb,
                               const GemmArgs& a, const GemmConfig& cfg, int splits,
                               float* ws) {
    const size_t mn = (size_t)a.M * (size_t)a.N;
    const int ks = a.K / splits;
    GemmBatchArgs b{};
    b.count = splits;
    b.tiles = (a.M / cfg.bm) * (a.N / cfg.bn);
    for (int z = 0; z < splits; z++) {
        GemmArgs q{};
        const long long k0 = (long long)z * ks;
        q.A = ta ? a.A + k0 * a.lda : a.A + k0;
        q.B = tb ? a.B + k0 : a.B + k0 * a.ldb;
        q.C = ws + (size_t)z * mn;
        q.M = a.M;
        q.N = a.N;
        q.K = ks;
        q.lda = a.lda;
        q.ldb = a.ldb;
        q.ldc = a.N;
        q.alpha = 1.0f;
        b.p[z] = q;
    }
    char name[96];
    snprintf(name, sizeof name, "forge_gemm_batch_%s_%s", gemm_ab(ta, tb), cfg.tag);
    void* args[] = {&b};
    FORGE_TRY(launch(rt, s, name, dim3((unsigned)(b.tiles * splits)), dim3(cfg.threads), 0,
                     args));
    const bool vec = a.N % 4 == 0;
    const size_t items = vec ? mn / 4 : mn;
    const unsigned grid = (unsigned)std::min<size_t>((items + 255) / 256, 8192);
    const float* P = ws;
    int sp = splits;
    GemmArgs e = a;
    void* rargs[] = {&P, &sp, &e};
    return launch(rt, s, vec ? "forge_gemm_splitk_reduce_v" : "forge_gemm_splitk_reduce_s",
                  dim3(grid), dim3(256), 0, rargs);
}

size_t sum_cols_scratch(size_t rows, size_t cols);
forge_status sum_cols_impl(forge_runtime* rt, forge_stream* s, const float* m, ColSumOut o,
                           size_t rows, size_t cols, float* scratch);

// Rows per wave (TM) of a tile: the eight-wave tile is 4 x 2 waves, the
// four-wave ones 2 x 2.
int tile_rows_per_wave(const GemmConfig& g) { return g.bm / (g.threads == 512 ? 4 : 2); }

// The epilogue's row statistics and column sums around one product launch
// (forge_gemm_epilogue row_parts_in, row_sumsq_out, col_sums_*).  On an
// unguarded tile the _s kernel forms the row scales from row_parts_in
// itself, writes row_sumsq_out and one partial row of column sums per
// wave-row of TM rows; on the guarded and split-K paths a small kernel forms
// the divisors first (row_d) and row_sumsq_out / the column sums are taken
// from C after the product.  The column sums end with one final pass that
// also applies the parameter's SGD step.  `ws` is the workspace that follows
// what the product itself uses.
struct GemmStatsWork {
    bool col = false, col_from_c = false, sq_from_c = false;
    float* col_part = nullptr;
    size_t col_rows = 0;
    float* chunk_scratch = nullptr;
};

size_t gemm_stats_floats(const forge_gemm_epilogue* ep, const GemmArgs& a, bool xtile,
                         const GemmConfig& cfg) {
    if (!gemm_has_stats(ep)) return 0;
    const size_t M = (size_t)a.M, N = (size_t)a.N;
    size_t n = 0;
    if (a.row_part && !xtile) n += M;
    if (ep->col_sums_out.ptr || ep->col_sums_param.ptr) {
        const size_t rows = xtile ? M / (size_t)tile_rows_per_wave(cfg) : M;
        if (xtile) n += rows * N;
        n += sum_cols_scratch(rows, N);
    }
    return n;
}

forge_status gemm_stats_prepare(forge_runtime* rt, forge_stream* s, const forge_gemm_epilogue* ep,
                                GemmArgs& a, bool xtile, const GemmConfig& cfg, float* ws,
                                GemmStatsWork* w) {
    if (!gemm_has_stats(ep)) return FORGE_OK;
    const size_t M = (size_t)a.M, N = (size_t)a.N;
    if (a.row_part && !xtile) {
        float* d = ws;
        ws += M;
        int m = a.M, parts = a.row_parts, n = a.row_n;
        float eps = a.row_eps;
        FORGE_TRY(launch_args(rt, s, "forge_row_rms_parts", dim3((unsigned)((M + 255) / 256)),
                              dim3(256), 0, (const float*)a.row_part, parts, m, n, eps, d));
        a.row_d = d;
        a.row_part = nullptr;
    }
    if (a.row_sq && !xtile) {
        a.row_sq = nullptr;
        w->sq_from_c = true;
    }
    if (ep->col_sums_out.ptr || ep->col_sums_param.ptr) {
        w->col = true;
        if (xtile) {
            w->col_rows = M / (size_t)tile_rows_per_wave(cfg);
            w->col_part = ws;
            ws += w->col_rows * N;
            a.col_part = w->col_part;
        } else {
            w->col_from_c = true;
            w->col_rows = M;
        }
        w->chunk_scratch = ws;
    }
    return FORGE_OK;
}

forge_status gemm_stats_finish(forge_runtime* rt, forge_stream* s, const forge_gemm_epilogue* ep,
                               const GemmArgs& a, const GemmStatsWork& w) {
    if (w.sq_from_c) {
        int m = a.M, n = a.N;
        long long ldc = a.ldc;
        const size_t parts = (size_t)((a.N + 31) / 32);
        FORGE_TRY(launch_args(rt, s, "forge_row_sq_parts",
                              dim3((unsigned)((parts * (size_t)a.M + 255) / 256)), dim3(256), 0,
                              (const float*)a.C, ldc, m, n, ep->row_sumsq_out.ptr));
    }
    if (w.col) {
        // C is dense (ldc == N) for every product here.
        const float* m = w.col_from_c ? a.C : w.col_part;
        return sum_cols_impl(rt, s, m,
                             ColSumOut{ep->col_sums_out.ptr, ep->col_sums_param.ptr,
                                       ep->col_sums_lr},
                             w.col_rows, (size_t)a.N, w.chunk_scratch);
    }
    return FORGE_OK;
}

// Column sums of no rows are zero and leave the parameter as it is; there
// are no rows to take statistics of.
forge_status gemm_stats_empty(forge_runtime* rt, forge_stream* s, const forge_gemm_epilogue* ep,
                              size_t N) {
    if (ep && ep->col_sums_out.ptr && N)
        return forge_fill(rt, s, forge_slice{ep->col_sums_out.ptr, N}, 0.0f);
    return FORGE_OK;
}

forge_status gemm_dispatch(forge_runtime* rt, forge_stream* s, int ta, int tb, forge_slice A,
                           forge_slice B, forge_slice C, size_t M, size_t N, size_t K,
                           const forge_gemm_epilogue* ep, bool plain_name) {
    GemmArgs a{};
    bool aligned = false;
    FORGE_TRY(gemm_args(ta, tb, A, B, C, M, N, K, ep, &a, &aligned));
    if (M == 0 || N == 0) return gemm_stats_empty(rt, s, ep, N);
    const GemmConfig* split_cfg = nullptr;
    const int splits = choose_splits(rt, ta, tb, M, N, K, aligned, &split_cfg);
    const GemmKind kind = ep && ep->row_sub.ptr        ? GemmKind::RowSub
                          : gemm_has_stats(ep)            ? GemmKind::Stats
                          : plain_name && !ta && !tb ? GemmKind::Plain
                                                     : GemmKind::Epilogue;
    const GemmPlan plan = splits > 1 ? GemmPlan{split_cfg, 0}
                                     : choose_gemm(rt, ta, tb, M, N, K, aligned, kind);
    const GemmConfig& cfg = *plan.cfg;
    const bool xtile = splits == 1 && &cfg != &kGuard64;
    const size_t split_floats = splits > 1 ? (size_t)splits * M * N : 0;
    const size_t stats_floats = gemm_stats_floats(ep, a, xtile, cfg);
    float* ws = nullptr;
    if (split_floats + stats_floats) FORGE_TRY(workspace(rt, s, split_floats + stats_floats, &ws));
    GemmStatsWork w;
    FORGE_TRY(gemm_stats_prepare(rt, s, ep, a, xtile, cfg, ws ? ws + split_floats : nullptr, &w));
    if (splits > 1) {
        FORGE_TRY(gemm_split_launch(rt, s, ta, tb, a, cfg, splits, ws));
    } else {
        char name[96];
        // The guarded tile has no statistics instance: its fused kernel
        // divides by row_d and subtracts row_sub per element, and the sums
        // come from C.
        const bool stats_kind = kind == GemmKind::Stats || kind == GemmKind::RowSub;
        gemm_kernel_name(name, sizeof name, xtile || !stats_kind ? kind : GemmKind::Epilogue, ta,
                         tb, cfg);
        size_t shmem = 0;
        if (plan.cap) FORGE_TRY(occupancy_cap_shmem(rt, name, plan.cap, &shmem));
        unsigned tiles = (unsigned)(((M + cfg.bm - 1) / cfg.bm) * ((N + cfg.bn - 1) / cfg.bn));
        void* args[] = {&a};
        FORGE_TRY(launch(rt, s, name, dim3(tiles), dim3(cfg.threads), shmem, args));
    }
    return gemm_stats_finish(rt, s, ep, a, w);
}

const char* binop_name(forge_binary_op op) {
    switch (op) {
    case FORGE_ADD: return "add";
    case FORGE_SUB: return "sub";
    case FORGE_MUL: return "mul";
    case FORGE_DIV: return "div";
    }
    return nullptr;
}

const char* map_name(forge_map_op op) {
    switch (op) {
    case FORGE_MAP_SCALE: return "scale";
    case FORGE_MAP_ADD: return "add";
    case FORGE_MAP_GELU: return "gelu";
    case FORGE_MAP_GELU_D: return "gelu_d";
    case FORGE_MAP_RELU: return "relu";
    case FORGE_MAP_RELU_D: return "relu_d";
    case FORGE_MAP_SILU: return "silu";
    case FORGE_MAP_SILU_D: return "silu_d";
    case FORGE_MAP_EXP_SHIFT: return "exp_shift";
    case FORGE_MAP_HALF_SQ: return "half_sq";
    case FORGE_MAP_IDENTITY: return "identity";
    }
    return nullptr;
}

// Elements per lane of the register path for `cols` (0 = use the loop path).
int row_vpt(size_t cols, bool aligned) {
    if (!aligned || cols % 4 != 0 || cols == 0) return 0;
    for (int v : {1, 2, 4, 8, 16})
        if (cols <= (size_t)v * 256) return v;
    return 0;
}

// Column sums of m [rows, cols] into out [cols].  Matrices of at most 512
// rows take one launch of forge_sum_cols_final (about 3 us on MI355X up to
// that height, latency-bound); taller ones first reduce chunks of rows into
// partial rows, then sum the partial rows with forge_sum_cols_final.  The
// first pass is forge_sum_cols_p<loads> when m, the outputs and the columns
// allow float4 throughout, else forge_sum_cols_v/_s (up to about 8192
// workgroups, >= 16 rows per chunk).  The chunking depends only on the
// shape, so the result is deterministic.
constexpr int SUMCOL_FINAL_MAX_ROWS = 512;
constexpr int SUMCOL_FINAL_V_THREADS = 256;  // elementwise.hpp SUMCOL_FINAL_V_THREADS
constexpr int SUMCOL_FINAL_V_COLS = 16;      // elementwise.hpp SUMCOL_FINAL_V_COLS

size_t sum_cols_chunks(size_t rows, size_t cols, bool vec) {
    if (rows <= (size_t)SUMCOL_FINAL_MAX_ROWS) return 1;
    size_t per_block = vec ? 256 : 64;
    size_t gx = (cols + per_block - 1) / per_block;
    size_t want = std::max<size_t>(1, 8192 / std::max<size_t>(1, gx));
    size_t by_rows = (rows + 15) / 16;
    return std::max<size_t>(2, std::min(want, std::min(by_rows, (size_t)SUMCOL_FINAL_MAX_ROWS)));
}

bool sum_cols_vec(const float* m, size_t cols) { return aligned16(m) && cols % 4 == 0; }

// First pass of the float4 column sums (forge_sum_cols_p<loads>,
// elementwise.hpp): workgroups of 64 columns by `rpc` rows, each lane
// `loads` float4 loads in flight, about SUMCOL_PART_TARGET workgroups in
// all and at most SUMCOL_PART_MAX_CHUNKS partial rows, so that
// forge_sum_cols_final_v adds them in one round of loads.
// $OXFORGE_SUMCOL_LOADS (4, 8 or 16) and $OXFORGE_SUMCOL_BLOCKS override the
// two choices (tuning knobs).  On MI355X a sweep of 4/8/16 loads by
// 256-2048 workgroups kept [4096,1024] at 7.4-8.3 us (two dependent
// launches); 16 loads by 512 is within 1% of the best there and at
// [4096,2048], 3-4% behind it at [65536,1024] and [4096,8192].
constexpr int SUMCOL1_COLS = 64;   // elementwise.hpp SUMCOL1_COLS
constexpr int SUMCOL1_SLOTS = 16;  // elementwise.hpp SUMCOL1_SLOTS
constexpr size_t SUMCOL_PART_TARGET = 512;
constexpr size_t SUMCOL_PART_MAX_CHUNKS = 256;

struct SumColsPart {
    int loads = 16;
    int rpc = 0;
    size_t chunks = 0;
};

long env_knob(const char* name) {
    const char* v = getenv(name);
    return v ? strtol(v, nullptr, 10) : 0L;
}

SumColsPart sum_cols_part_plan(size_t rows, size_t cols) {
    static const long env_loads = env_knob("OXFORGE_SUMCOL_LOADS");
    static const long env_blocks = env_knob("OXFORGE_SUMCOL_BLOCKS");
    SumColsPart p;
    if (env_loads == 4 || env_loads == 8 || env_loads == 16) p.loads = (int)env_loads;
    const size_t target = env_blocks > 0 ? (size_t)env_blocks : SUMCOL_PART_TARGET;
    const size_t gx = (cols + SUMCOL1_COLS - 1) / SUMCOL1_COLS;
    const size_t batch = (size_t)SUMCOL1_SLOTS * p.loads;
    const size_t batches = (rows + batch - 1) / batch;
    size_t chunks = std::max<size_t>(1, target / gx);
    chunks = std::min(chunks, std::min(batches, SUMCOL_PART_MAX_CHUNKS));
    const size_t per = (batches + chunks - 1) / chunks;
    p.rpc = (int)(per * batch);
    p.chunks = (rows + (size_t)p.rpc - 1) / (size_t)p.rpc;
    return p;
}

// Floats of scratch sum_cols_impl needs for this shape.
size_t sum_cols_scratch(size_t rows, size_t cols) {
    size_t chunks = sum_cols_chunks(rows, cols, true);
    size_t chunks_s = sum_cols_chunks(rows, cols, false);
    size_t c = std::max(chunks, chunks_s);
    if (c > 1) c = std::max(c, sum_cols_part_plan(rows, cols).chunks);
    return c > 1 ? c * cols : 0;
}

// Final column-sum pass over a matrix of at most SUMCOL_FINAL_MAX_ROWS rows:
// float4 columns when m, the outputs and the parameter are 16-byte aligned
// and cols % 4 == 0.
bool sum_cols_final_vec(const float* m, const ColSumOut& o, int cols) {
    return aligned16(m) && (!o.out || aligned16(o.out)) && (!o.param || aligned16(o.param)) &&
           cols % 4 == 0;
}

forge_status sum_cols_final_launch(forge_runtime* rt, forge_stream* s, const float* m,
                                   ColSumOut o, int rows, int cols) {
    if (sum_cols_final_vec(m, o, cols))
        return launch_args(rt, s, "forge_sum_cols_final_v",
                           dim3((unsigned)((cols + SUMCOL_FINAL_V_COLS - 1) / SUMCOL_FINAL_V_COLS)),
                           dim3(SUMCOL_FINAL_V_THREADS), 0, m, o, rows, cols);
    return launch_args(rt, s, "forge_sum_cols_final", dim3((unsigned)((cols + 63) / 64)),
                       dim3(1024), 0, m, o, rows, cols);
}

// scratch: sum_cols_scratch(rows, cols) floats that do not overlap m or the
// outputs.
forge_status sum_cols_impl(forge_runtime* rt, forge_stream* s, const float* m, ColSumOut o,
                           size_t rows, size_t cols, float* scratch) {
    if (cols == 0) return FORGE_OK;
    int c = (int)cols;
    const bool vec = sum_cols_vec(m, cols);
    size_t chunks = sum_cols_chunks(rows, cols, vec);
    if (chunks == 1) return sum_cols_final_launch(rt, s, m, o, (int)rows, c);
    if (sum_cols_final_vec(m, o, c)) {
        // float4 first pass; a single chunk stores the sums itself.
        const SumColsPart p = sum_cols_part_plan(rows, cols);
        char name[40];
        snprintf(name, sizeof name, "forge_sum_cols_p%d", p.loads);
        int r = (int)rows;
        const unsigned gx = (unsigned)((cols + SUMCOL1_COLS - 1) / SUMCOL1_COLS);
        FORGE_TRY(launch_args(rt, s, name, dim3(gx, (unsigned)p.chunks), dim3(256), 0, m, scratch,
                              o, r, c, p.rpc));
        if (p.chunks == 1) return FORGE_OK;
        return sum_cols_final_launch(rt, s, scratch, o, (int)p.chunks, c);
    }
    int rpc = (int)((rows + chunks - 1) / chunks);
    chunks = (rows + rpc - 1) / rpc;
    int r = (int)rows;
    unsigned gx = (unsigned)((cols + (vec ? 255 : 63)) / (vec ? 256 : 64));
    FORGE_TRY(launch_args(rt, s, vec ? "forge_sum_cols_v" : "forge_sum_cols_s",
                          dim3(gx, (unsigned)chunks), dim3(256), 0, m, scratch, r, c, rpc));
    return sum_cols_final_launch(rt, s, scratch, o, (int)chunks, c);
}


// Workgroups of the dgamma/dbeta partial pass of the norm backward kernels:
// $OXFORGE_NORM_BWD_BLOCKS when set (a tuning knob), else per_cu per CU.
unsigned norm_bwd_blocks(forge_runtime* rt, int per_cu) {
    static const long env = [] {
        const char* v = getenv("OXFORGE_NORM_BWD_BLOCKS");
        return v ? strtol(v, nullptr, 10) : 0L;
    }();
    if (env > 0) return (unsigned)env;
    return (unsigned)(std::max(64, rt->cu_count) * per_cu);
}

// Shared launcher of the six row kernels.  For the norm backward kernels
// with dgamma/dbeta requested, the partial rows land in the stream's
// workspace and are summed by sum_cols_impl; with `scratch` given they land
// there instead (scratch_len floats, nothing is allocated) and a shape that
// needs more is FORGE_EINVAL.
// The SGD step of the norm's own parameters, applied by the final column-sum
// pass of its backward (gamma/beta null: no step).
struct NormSgd {
    float* gamma = nullptr;
    float* beta = nullptr;
    float lr = 0.0f;
};

// Elements from which the norm backward kernels store non-temporally.
constexpr long long kNormBwdNtMin = 8ll << 20;

forge_status row_launch(forge_runtime* rt, forge_stream* s, const char* op, RowArgs a,
                        float* dgamma, float* dbeta, float* scratch = nullptr,
                        size_t scratch_len = 0, NormSgd sgd = NormSgd()) {
    if (a.rows == 0 || a.cols == 0) {
        // No rows: zero gradients, and the SGD step leaves the parameters.
        // Empty rows: each row dot is zero.
        if (dgamma) FORGE_TRY(forge_fill(rt, s, forge_slice{dgamma, (size_t)a.cols}, 0.0f));
        if (dbeta) FORGE_TRY(forge_fill(rt, s, forge_slice{dbeta, (size_t)a.cols}, 0.0f));
        if (a.dot && a.rows > 0)
            FORGE_TRY(forge_fill(rt, s, forge_slice{a.dot, (size_t)a.rows}, 0.0f));
        return FORGE_OK;
    }
    // The forward kernels store non-temporally at every size: at
    // [4096,1024] softmax 7.29 -> 6.32 us, RMSNorm 7.86 -> 7.15 us, and
    // LayerNorm (with gamma/beta staged in LDS) 7.65-7.68 -> 6.89-6.90 us,
    // 14.8 -> 13.4 us at [4096,2048].  The backward kernels, like
    // everything else, store non-temporally from 64 MiB on, the norm
    // backward kernels from 32 MiB: at [4096,2048] (with dgamma/dbeta) the
    // LayerNorm backward took 25.3 against 27.2 us with them and the RMSNorm
    // backward 22.6 against 24.6 us, at [4096,1024] 14.9 against 14.5 and
    // 13.4 against 13.0 us; the softmax backward was 0.3 us slower at
    // [4096,1024].
    a.nt_stores = (strcmp(op, "softmax") == 0 || strcmp(op, "rms_norm") == 0 ||
                   strcmp(op, "layer_norm") == 0 ||
                   (strstr(op, "norm_bwd") && (long long)a.rows * a.cols >= kNormBwdNtMin))
                      ? 1 : 0;
    a.lds_params =
        (strcmp(op, "layer_norm") == 0 && (long long)a.rows * a.cols < kRowLdsParamsMax) ? 1 : 0;
    const ColSumOut og{dgamma, sgd.gamma, sgd.lr}, ob{dbeta, sgd.beta, sgd.lr};
    const bool want_g = dgamma || sgd.gamma, want_b = dbeta || sgd.beta;
    bool aligned = aligned16(a.x) && aligned16(a.y) && (!a.dy || aligned16(a.dy)) &&
                   (!a.gamma || aligned16(a.gamma)) && (!a.beta || aligned16(a.beta)) &&
                   (!a.dsub || aligned16(a.dsub));
    // The row dot (norm backward): the register path's _d instances; the
    // looping path takes it at run time.
    const char* dsuf = a.dot ? "_d" : "";
    int vpt = row_vpt((size_t)a.cols, aligned);
    const bool partials = want_g || want_b;
    if (partials && vpt > 8) vpt = 0;  // register path with partials: <= 8 float4
    char name[80];
    // Waves per workgroup: the register partial kernels use ROW_PARTIAL_WAVES
    // (one LDS-combined partial row per workgroup); everything else ROW_WAVES.
    // At 4 float4 per lane and at least 256 rows per CU the partial kernel
    // runs 4 waves per workgroup (the _p4 instance).
    const bool p4 = partials && vpt == 4 && (size_t)a.rows >= 256 * (size_t)rt->cu_count;
    const int waves = (partials && vpt) ? (p4 ? 4 : ROW_PARTIAL_WAVES) : ROW_WAVES;
    unsigned blocks_needed = (unsigned)((a.rows + waves - 1) / waves);
    unsigned grid;
    size_t shmem = 0;
    size_t prow = 0;
    float* ws = nullptr;
    if (partials) {
        // One partial row per workgroup (register path) or per wave (loop).
        // The four-wave LayerNorm backward runs two workgroups per CU:
        // [65536,1024] 131.8 against 132.8 us with one (three runs each;
        // grids that are not a multiple of the CU count are 4-20% slower).
        // RMSNorm, 1.5% slower with two, keeps one.
        const int per_cu = (p4 && strcmp(op, "layer_norm_bwd") == 0) ? 2 : 1;
        grid = std::min<unsigned>(blocks_needed, norm_bwd_blocks(rt, per_cu));
        prow = vpt ? grid : (size_t)grid * ROW_WAVES;
        size_t per = prow * (size_t)a.cols;
        const size_t need = per * 2 + sum_cols_scratch(prow, (size_t)a.cols);
        if (scratch) {
            if (need > scratch_len)
                return fail(FORGE_EINVAL,
                            "%s with dgamma/dbeta at [%d, %d] needs %zu floats of scratch; the "
                            "no-allocation scratch holds %zu",
                            op, a.rows, a.cols, need, scratch_len);
            ws = scratch;
        } else {
            FORGE_TRY(workspace(rt, s, need, &ws));
        }
        a.pgamma = want_g ? ws : nullptr;
        a.pbeta = want_b ? ws + per : nullptr;
        if (vpt) shmem = (size_t)waves * (size_t)a.cols * sizeof(float);
        if (vpt)
            snprintf(name, sizeof name, "forge_row_%s_v%d_p%s%s", op, vpt, p4 ? "4" : "", dsuf);
        else snprintf(name, sizeof name, "forge_row_%s_loop", op);
    } else {
        grid = std::min<unsigned>(blocks_needed, 1u << 20);
        if (vpt) snprintf(name, sizeof name, "forge_row_%s_v%d%s", op, vpt, dsuf);
        else snprintf(name, sizeof name, "forge_row_%s_loop", op);
    }
    if (shmem > rt->lds_bytes)
        return fail(FORGE_EINVAL, "row kernel needs %zu B of LDS, the device has %zu", shmem,
                    rt->lds_bytes);
    void* args[] = {&a};
    FORGE_TRY(launch(rt, s, name, dim3(grid), dim3(waves * 64), shmem, args));
    float* chunk_scratch = ws ? ws + 2 * prow * (size_t)a.cols : nullptr;
    if (want_g && want_b && sum_cols_chunks(prow, (size_t)a.cols, true) == 1) {
        // Both column sums fit one final pass: one launch for the pair.
        int r = (int)prow, c = a.cols;
        if (sum_cols_final_vec(a.pgamma, og, c) && sum_cols_final_vec(a.pbeta, ob, c))
            return launch_args(rt, s, "forge_sum_cols_final2_v",
                               dim3((unsigned)((c + SUMCOL_FINAL_V_COLS - 1) / SUMCOL_FINAL_V_COLS), 2),
                               dim3(SUMCOL_FINAL_V_THREADS), 0, (const float*)a.pgamma, og,
                               (const float*)a.pbeta, ob, r, c);
        unsigned gfinal = (unsigned)((a.cols + 63) / 64);
        return launch_args(rt, s, "forge_sum_cols_final2", dim3(gfinal, 2), dim3(1024), 0,
                           (const float*)a.pgamma, og, (const float*)a.pbeta, ob, r, c);
    }
    if (want_g)
        FORGE_TRY(sum_cols_impl(rt, s, a.pgamma, og, prow, (size_t)a.cols, chunk_scratch));
    if (want_b)
        FORGE_TRY(sum_cols_impl(rt, s, a.pbeta, ob, prow, (size_t)a.cols, chunk_scratch));
    return FORGE_OK;
}

forge_status check_rows(size_t rows, size_t cols) {
    if (!fits_int(rows) || !fits_int(cols)) return fail(FORGE_EINVAL, "rows/cols exceed 2^31-1");
    return FORGE_OK;
}

}  // namespace

extern "C" forge_status forge_gemm_f32(forge_runtime* rt, forge_stream* s, forge_slice A,
                                       forge_slice B, forge_slice C, size_t M, size_t N,
                                       size_t K) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    return gemm_dispatch(rt, s, 0, 0, A, B, C, M, N, K, nullptr, true);
}

extern "C" forge_status forge_gemm_ex_f32(forge_runtime* rt, forge_stream* s, int trans_a,
                                          int trans_b, forge_slice A, forge_slice B, forge_slice C,
                                          size_t M, size_t N, size_t K,
                                          const forge_gemm_epilogue* ep) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    return gemm_dispatch(rt, s, trans_a != 0, trans_b != 0, A, B, C, M, N, K, ep, false);
}

// "<tile>" or "<tile>@<n>" (at most n workgroups per CU; 0 = no limit).
forge_status split_tile_tag(const char* in, char* tag, size_t cap_bytes, int* cap) {
    const char* at = strchr(in, '@');
    const size_t len = at ? (size_t)(at - in) : strlen(in);
    if (len >= cap_bytes) return fail(FORGE_EINVAL, "bad tile tag %s", in);
    memcpy(tag, in, len);
    tag[len] = 0;
    *cap = 0;
    if (at && (sscanf(at + 1, "%d", cap) != 1 || *cap < 1 || *cap > 16))
        return fail(FORGE_EINVAL, "bad occupancy cap in %s", in);
    return FORGE_OK;
}

extern "C" forge_status forge_gemm_f32_tile(forge_runtime* rt, forge_stream* s,
                                            const char* tile_tag_in, forge_slice A,
                                            forge_slice B, forge_slice C, size_t M, size_t N,
                                            size_t K) {
    if (!rt || !tile_tag_in) return fail(FORGE_EINVAL, "null argument");
    char tile_tag[32];
    int cap = 0;
    FORGE_TRY(split_tile_tag(tile_tag_in, tile_tag, sizeof tile_tag, &cap));
    unsigned bm = 0, bn = 0, bk = 0;
    unsigned threads = 256;
    bool guarded = false;
    char tail[8] = {0};
    if (sscanf(tile_tag, "%ux%ux%u_%7s", &bm, &bn, &bk, tail) != 4 || bm == 0 || bn == 0 ||
        bk == 0)
        return fail(FORGE_EINVAL, "bad tile tag %s", tile_tag);
    if (strcmp(tail, "x") == 0) {
        // Four-wave instance <BM>x<BN>x<BK>_x.
    } else if (strcmp(tail, "x8") == 0) {
        threads = 512;  // eight-wave instance
    } else if (strcmp(tail, "2x2_g") == 0) {
        guarded = true;
    } else {
        return fail(FORGE_EINVAL, "bad tile tag %s", tile_tag);
    }
    if (!fits_int(M) || !fits_int(N) || !fits_int(K))
        return fail(FORGE_EINVAL, "gemm dimensions exceed 2^31-1");
    FORGE_TRY(need(A, M * K, "gemm A"));
    FORGE_TRY(need(B, K * N, "gemm B"));
    FORGE_TRY(need(C, M * N, "gemm C"));
    if (!guarded && (M % bm || N % bn || K % bk || !aligned16(A.ptr) ||
                     !aligned16(B.ptr) || !aligned16(C.ptr) || K % 4 || N % 4 ||
                     (long long)K > kUnguardedMaxPitch || (long long)N > kUnguardedMaxPitch))
        return fail(FORGE_EINVAL, "shape %zux%zux%zu does not fit unguarded tile %s", M, N, K,
                    tile_tag);
    if (M == 0 || N == 0) return FORGE_OK;
    GemmArgs a{};
    a.A = A.ptr;
    a.B = B.ptr;
    a.C = C.ptr;
    a.M = (int)M;
    a.N = (int)N;
    a.K = (int)K;
    a.lda = (long long)K;
    a.ldb = (long long)N;
    a.ldc = (long long)N;
    a.alpha = 1.0f;
    char name[96];
    snprintf(name, sizeof name, "forge_gemm_nn_%s", tile_tag);
    size_t shmem = 0;
    if (cap) FORGE_TRY(occupancy_cap_shmem(rt, name, cap, &shmem));
    unsigned tiles = (unsigned)(((M + bm - 1) / bm) * ((N + bn - 1) / bn));
    void* args[] = {&a};
    return launch(rt, s, name, dim3(tiles), dim3(threads), shmem, args);
}

extern "C" forge_status forge_gemm_f32_split(forge_runtime* rt, forge_stream* s,
                                             const char* tile_tag, int splits, forge_slice A,
                                             forge_slice B, forge_slice C, size_t M, size_t N,
                                             size_t K) {
    if (!rt || !tile_tag) return fail(FORGE_EINVAL, "null argument");
    const GemmConfig* cfg = nullptr;
    for (const GemmConfig* c : kUnguarded)
        if (c != &kTile128x256 && strcmp(c->tag, tile_tag) == 0) cfg = c;
    if (!cfg) return fail(FORGE_EINVAL, "tile %s has no batched instance", tile_tag);
    if (splits < 1 || splits > GEMM_BATCH_MAX)
        return fail(FORGE_EINVAL, "splits must be in [1, %d]", GEMM_BATCH_MAX);
    GemmArgs a{};
    bool aligned = false;
    FORGE_TRY(gemm_args(0, 0, A, B, C, M, N, K, nullptr, &a, &aligned));
    if (!aligned || M % cfg->bm || N % cfg->bn || K % ((size_t)splits * cfg->bk))
        return fail(FORGE_EINVAL, "shape %zux%zux%zu does not fit tile %s with %d splits", M, N,
                    K, tile_tag, splits);
    if (M == 0 || N == 0) return FORGE_OK;
    float* ws = nullptr;
    FORGE_TRY(workspace(rt, s, (size_t)splits * M * N, &ws));
    return gemm_split_launch(rt, s, 0, 0, a, *cfg, splits, ws);
}

extern "C" forge_status forge_gemm_ex_f32_tile(forge_runtime* rt, forge_stream* s,
                                               const char* tile_tag_in, int trans_a, int trans_b,
                                               forge_slice A, forge_slice B, forge_slice C,
                                               size_t M, size_t N, size_t K,
                                               const forge_gemm_epilogue* ep) {
    if (!rt || !tile_tag_in) return fail(FORGE_EINVAL, "null argument");
    char tile_tag[32];
    int cap = 0;
    FORGE_TRY(split_tile_tag(tile_tag_in, tile_tag, sizeof tile_tag, &cap));
    const GemmConfig* cfg = nullptr;
    if (strcmp(kGuard64.tag, tile_tag) == 0) cfg = &kGuard64;
    for (const GemmConfig* c : kUnguarded)
        if (c != &kTile128x256 && strcmp(c->tag, tile_tag) == 0) cfg = c;
    if (!cfg) return fail(FORGE_EINVAL, "tile %s has no epilogue instance", tile_tag);
    GemmArgs a{};
    bool aligned = false;
    FORGE_TRY(gemm_args(trans_a, trans_b, A, B, C, M, N, K, ep, &a, &aligned));
    if (cfg != &kGuard64 &&
        (!aligned || M % cfg->bm || N % cfg->bn || K % (size_t)cfg->bk))
        return fail(FORGE_EINVAL, "shape %zux%zux%zu does not fit unguarded tile %s", M, N, K,
                    tile_tag);
    if (M == 0 || N == 0) return gemm_stats_empty(rt, s, ep, N);
    const bool xtile = cfg != &kGuard64;
    float* ws = nullptr;
    const size_t stats_floats = gemm_stats_floats(ep, a, xtile, *cfg);
    if (stats_floats) FORGE_TRY(workspace(rt, s, stats_floats, &ws));
    GemmStatsWork w;
    FORGE_TRY(gemm_stats_prepare(rt, s, ep, a, xtile, *cfg, ws, &w));
    char name[96];
    snprintf(name, sizeof name, "forge_gemm_%s_%s_%s", gemm_ab(trans_a, trans_b), cfg->tag,
             !xtile                        ? "e"
             : ep && ep->row_sub.ptr       ? "r"
             : gemm_has_stats(ep)          ? "s"
                                           : "e");
    size_t shmem = 0;
    if (cap) FORGE_TRY(occupancy_cap_shmem(rt, name, cap, &shmem));
    const unsigned tiles =
        (unsigned)(((M + cfg->bm - 1) / cfg->bm) * ((N + cfg->bn - 1) / cfg->bn));
    void* args[] = {&a};
    FORGE_TRY(launch(rt, s, name, dim3(tiles), dim3(cfg->threads), shmem, args));
    return gemm_stats_finish(rt, s, ep, a, w);
}

extern "C" forge_status forge_gemm_kernel_name(forge_runtime* rt, int trans_a, int trans_b,
                                               size_t M, size_t N, size_t K, int fused,
                                               char* name, size_t cap) {
    if (!rt || !name || cap == 0) return fail(FORGE_EINVAL, "null argument");
    if (!fits_int(M) || !fits_int(N) || !fits_int(K))
        return fail(FORGE_EINVAL, "gemm dimensions exceed 2^31-1");
    const int ta = trans_a ? 1 : 0, tb = trans_b ? 1 : 0;
    const long long lda = ta ? (long long)M : (long long)K;
    const long long ldb = tb ? (long long)K : (long long)N;
    const bool aligned = lda % 4 == 0 && ldb % 4 == 0 && lda <= kUnguardedMaxPitch &&
                         ldb <= kUnguardedMaxPitch;
    const GemmConfig* split_cfg = nullptr;
    const int splits = choose_splits(rt, ta, tb, M, N, K, aligned, &split_cfg);
    char kernel[96];
    int n = 0;
    if (splits > 1) {
        gemm_kernel_name(kernel, sizeof kernel, GemmKind::Batch, ta, tb, *split_cfg);
        n = snprintf(name, cap, "%s/split%d", kernel, splits);
    } else {
        const GemmKind kind = !fused && !ta && !tb ? GemmKind::Plain : GemmKind::Epilogue;
        const GemmPlan plan = choose_gemm(rt, ta, tb, M, N, K, aligned, kind);
        gemm_kernel_name(kernel, sizeof kernel, kind, ta, tb, *plan.cfg);
        n = plan.cap ? snprintf(name, cap, "%s@%d", kernel, plan.cap)
                     : snprintf(name, cap, "%s", kernel);
    }
    if (n < 0 || (size_t)n >= cap) return fail(FORGE_EINVAL, "name buffer of %zu bytes too small", cap);
    return FORGE_OK;
}

// Copies count operands of rows x cols (row-major, pitch cols) side by side
// into dst [rows, count * cols] (concatenation along the columns).
static forge_status concat_cols(forge_runtime* rt, forge_stream* s, float* dst,
                                const forge_slice* src, size_t count, size_t rows, size_t cols) {
    for (size_t z = 0; z < count; z++)
        HIP_TRY(hipMemcpy2DAsync(dst + z * cols, count * cols * sizeof(float), src[z].ptr,
                                 cols * sizeof(float), cols * sizeof(float), rows,
                                 hipMemcpyDeviceToDevice, pick(rt, s)->stream));
    return FORGE_OK;
}

extern "C" forge_status forge_gemm_sum_f32(forge_runtime* rt, forge_stream* s, int trans_a,
                                           int trans_b, size_t count, const forge_slice* A,
                                           const forge_slice* B, forge_slice C, size_t M,
                                           size_t N, size_t K, const forge_gemm_epilogue* ep) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (count < 1 || count > 3) return fail(FORGE_EINVAL, "gemm_sum count %zu is not 1-3", count);
    if (!A || !B) return fail(FORGE_EINVAL, "gemm_sum operands are null");
    const int ta = trans_a != 0, tb = trans_b != 0;
    GemmArgs a{};
    bool aligned = true;
    for (size_t z = 0; z < count; z++) {
        GemmArgs az{};
        bool al = false;
        FORGE_TRY(gemm_args(ta, tb, A[z], B[z], C, M, N, K, ep, &az, &al));
        aligned = aligned && al;
        if (z == 0) a = az;
    }
    // One product, or an empty one (no rows, columns or K: the epilogue of
    // zeros), is the plain fused product.
    if (count == 1 || M == 0 || N == 0 || K == 0)
        return gemm_dispatch(rt, s, ta, tb, A[0], B[0], C, M, N, K, ep, false);
    const size_t Kt = count * K;
    if (!fits_int(Kt)) return fail(FORGE_EINVAL, "gemm_sum K exceeds 2^31-1");
    // One launch over the K segments when an unguarded tile takes the whole
    // product unsplit, with no statistics in its epilogue; else the
    // operands are concatenated along K and the product runs as one GEMM.
    // Both give the result of forge_gemm_ex_f32 on the concatenation.
    if (M && N && aligned && K % 32 == 0 && !gemm_has_stats(ep)) {
        const GemmConfig* split_cfg = nullptr;
        if (choose_splits(rt, ta, tb, M, N, Kt, true, &split_cfg) == 1) {
            const GemmPlan plan = choose_gemm(rt, ta, tb, M, N, Kt, true, GemmKind::SegK);
            if (plan.cfg != &kGuard64) {
                const GemmConfig& cfg = *plan.cfg;
                a.K = (int)Kt;
                a.k_seg = (int)K;
                a.A1 = A[1].ptr;
                a.B1 = B[1].ptr;
                a.A2 = count > 2 ? A[2].ptr : nullptr;
                a.B2 = count > 2 ? B[2].ptr : nullptr;
                char name[96];
                gemm_kernel_name(name, sizeof name, GemmKind::SegK, ta, tb, cfg);
                size_t shmem = 0;
                if (plan.cap) FORGE_TRY(occupancy_cap_shmem(rt, name, plan.cap, &shmem));
                const unsigned tiles = (unsigned)((M / cfg.bm) * (N / cfg.bn));
                void* args[] = {&a};
                return launch(rt, s, name, dim3(tiles), dim3(cfg.threads), shmem, args);
            }
        }
    }
    // Concatenation along K: op(A) [M, K] segments side by side (rows of A
    // stacked when A is stored transposed), op(B) [K, N] segments stacked
    // (side by side when B is stored transposed).
    forge_slice ac{}, bc{};
    FORGE_TRY(forge_alloc(rt, Kt * M, &ac));
    FORGE_TRY(forge_alloc(rt, Kt * N, &bc));
    forge_status st = FORGE_OK;
    for (size_t z = 0; z < count && st == FORGE_OK; z++) {
        if (ta) st = forge_memcpy_d2d(rt, s, forge_slice{ac.ptr + z * K * M, K * M}, A[z], K * M);
        if (!tb && st == FORGE_OK)
            st = forge_memcpy_d2d(rt, s, forge_slice{bc.ptr + z * K * N, K * N}, B[z], K * N);
    }
    if (st == FORGE_OK && !ta) st = concat_cols(rt, s, ac.ptr, A, count, M, K);
    if (st == FORGE_OK && tb) st = concat_cols(rt, s, bc.ptr, B, count, N, K);
    if (st == FORGE_OK) st = gemm_dispatch(rt, s, ta, tb, ac, bc, C, M, N, Kt, ep, false);
    forge_recycle(rt, ac);
    forge_recycle(rt, bc);
    return st;
}

extern "C" forge_status forge_gemm_batch_f32(forge_runtime* rt, forge_stream* s, int trans_a,
                                             int trans_b, size_t M, size_t N, size_t K,
                                             size_t count, const forge_gemm_problem* problems) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (count > 0 && !problems) return fail(FORGE_EINVAL, "problems is null");
    GemmBatchArgs b{};
    bool all_aligned = true, stats = false;
    for (size_t z = 0; z < count; z++) {
        GemmArgs a{};
        bool aligned = false;
        FORGE_TRY(gemm_args(trans_a, trans_b, problems[z].A, problems[z].B, problems[z].C, M, N,
                            K, &problems[z].epilogue, &a, &aligned));
        all_aligned = all_aligned && aligned;
        stats = stats || gemm_has_stats(&problems[z].epilogue);
        if (z < (size_t)GEMM_BATCH_MAX) b.p[z] = a;
    }
    if (count == 0 || M == 0 || N == 0) return FORGE_OK;
    const GemmPlan plan =
        choose_gemm(rt, trans_a, trans_b, M, N, K, all_aligned, GemmKind::Batch, count);
    const GemmConfig& cfg = *plan.cfg;
    const GemmConfig* split_cfg = nullptr;
    // Shapes the single-product path splits in K are dispatched one by one,
    // so every product equals its forge_gemm_ex_f32 result bit for bit.
    const bool split = choose_splits(rt, trans_a, trans_b, M, N, K, all_aligned, &split_cfg) > 1;
    if (count > (size_t)GEMM_BATCH_MAX || &cfg == &kGuard64 || split || stats) {
        for (size_t z = 0; z < count; z++)
            FORGE_TRY(gemm_dispatch(rt, s, trans_a, trans_b, problems[z].A, problems[z].B,
                                    problems[z].C, M, N, K, &problems[z].epilogue, false));
        return FORGE_OK;
    }
    b.count = (int)count;
    b.tiles = (int)((M / cfg.bm) * (N / cfg.bn));
    char name[96];
    gemm_kernel_name(name, sizeof name, GemmKind::Batch, trans_a, trans_b, cfg);
    size_t shmem = 0;
    if (plan.cap) FORGE_TRY(occupancy_cap_shmem(rt, name, plan.cap, &shmem));
    void* args[] = {&b};
    return launch(rt, s, name, dim3((unsigned)(b.tiles * count)), dim3(cfg.threads), shmem,
                  args);
}

extern "C" forge_status forge_transpose_f32(forge_runtime* rt, forge_stream* s, forge_slice in,
                                            forge_slice out, size_t rows, size_t cols) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(in, rows * cols, "transpose in"));
    FORGE_TRY(need(out, rows * cols, "transpose out"));
    if (rows == 0 || cols == 0) return FORGE_OK;
    // 64x256 tiles when the shape divides, 64x64 otherwise, guarded 64x64
    // for edges and views not 16-byte aligned.
    const bool fast = aligned16(in.ptr) && aligned16(out.ptr) && rows % 64 == 0 && cols % 64 == 0;
    const bool wide = fast && cols % 256 == 0;
    const size_t tc = wide ? 256 : 64;
    unsigned tiles = (unsigned)(((rows + 63) / 64) * ((cols + tc - 1) / tc));
    int r = (int)rows, c = (int)cols;
    const char* name = wide ? "forge_transpose_w" : fast ? "forge_transpose" : "forge_transpose_g";
    return launch_args(rt, s, name, dim3(tiles), dim3(256), 0, (const float*)in.ptr, out.ptr, r, c);
}

extern "C" forge_status forge_softmax_rows(forge_runtime* rt, forge_stream* s, forge_slice x,
                                           size_t rows, size_t cols) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(x, rows * cols, "softmax x"));
    RowArgs a{x.ptr, x.ptr, nullptr, nullptr, nullptr, nullptr, nullptr, (int)rows, (int)cols, 0.f, 1.0f};
    return row_launch(rt, s, "softmax", a, nullptr, nullptr);
}

extern "C" forge_status forge_softmax_rows_bwd(forge_runtime* rt, forge_stream* s, forge_slice p,
                                               forge_slice g, forge_slice dx, size_t rows,
                                               size_t cols) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(p, rows * cols, "softmax_bwd p"));
    FORGE_TRY(need(g, rows * cols, "softmax_bwd g"));
    FORGE_TRY(need(dx, rows * cols, "softmax_bwd dx"));
    RowArgs a{p.ptr, dx.ptr, g.ptr, nullptr, nullptr, nullptr, nullptr, (int)rows, (int)cols, 0.f, 1.0f};
    return row_launch(rt, s, "softmax_bwd", a, nullptr, nullptr);
}

// y == x (in place) or y disjoint from x; partial overlap is rejected.
static forge_status check_out_of_place(forge_slice x, forge_slice y, size_t n, const char* what) {
    if (x.ptr == y.ptr) return FORGE_OK;
    const float *xb = x.ptr, *yb = y.ptr;
    if (yb < xb + n && xb < yb + n)
        return fail(FORGE_EINVAL, "%s: output overlaps the input without being it", what);
    return FORGE_OK;
}

extern "C" forge_status forge_layer_norm_rows_out(forge_runtime* rt, forge_stream* s,
                                                  forge_slice x, forge_slice y, forge_slice gamma,
                                                  forge_slice beta, size_t rows, size_t cols,
                                                  float eps) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(x, rows * cols, "layer_norm x"));
    FORGE_TRY(need(y, rows * cols, "layer_norm y"));
    FORGE_TRY(check_out_of_place(x, y, rows * cols, "layer_norm"));
    FORGE_TRY(need_opt(gamma, cols, "layer_norm gamma"));
    FORGE_TRY(need_opt(beta, cols, "layer_norm beta"));
    RowArgs a{x.ptr, y.ptr, nullptr, gamma.ptr, beta.ptr, nullptr, nullptr, (int)rows, (int)cols, eps, 1.0f};
    return row_launch(rt, s, "layer_norm", a, nullptr, nullptr);
}

extern "C" forge_status forge_layer_norm_rows(forge_runtime* rt, forge_stream* s, forge_slice x,
                                              forge_slice gamma, forge_slice beta, size_t rows,
                                              size_t cols, float eps) {
    return forge_layer_norm_rows_out(rt, s, x, x, gamma, beta, rows, cols, eps);
}

namespace {
forge_status layer_norm_bwd_impl(forge_runtime* rt, forge_stream* s, forge_slice x,
                                 forge_slice dy, forge_slice gamma, forge_slice dx,
                                 forge_slice dgamma, forge_slice dbeta, size_t rows, size_t cols,
                                 float eps, float* scratch, size_t scratch_len) {
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(x, rows * cols, "layer_norm_bwd x"));
    FORGE_TRY(need(dy, rows * cols, "layer_norm_bwd dy"));
    FORGE_TRY(need(dx, rows * cols, "layer_norm_bwd dx"));
    FORGE_TRY(need_opt(gamma, cols, "layer_norm_bwd gamma"));
    FORGE_TRY(need_opt(dgamma, cols, "layer_norm_bwd dgamma"));
    FORGE_TRY(need_opt(dbeta, cols, "layer_norm_bwd dbeta"));
    RowArgs a{x.ptr, dx.ptr, dy.ptr, gamma.ptr, nullptr, nullptr, nullptr, (int)rows, (int)cols, eps, 1.0f};
    return row_launch(rt, s, "layer_norm_bwd", a, dgamma.ptr, dbeta.ptr, scratch, scratch_len);
}
}  // namespace

extern "C" forge_status forge_layer_norm_bwd(forge_runtime* rt, forge_stream* s, forge_slice x,
                                             forge_slice dy, forge_slice gamma, forge_slice dx,
                                             forge_slice dgamma, forge_slice dbeta, size_t rows,
                                             size_t cols, float eps) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    return layer_norm_bwd_impl(rt, s, x, dy, gamma, dx, dgamma, dbeta, rows, cols, eps, nullptr,
                               0);
}

// The norm backward's row dot operands (forge_*_norm_bwd_sgd_dot): sub
// [rows, cols] is disjoint from dx, dot [rows] from every matrix operand.
static forge_status row_dot_args(forge_slice x, forge_slice dy, forge_slice dx, forge_slice sub,
                                 forge_slice dot, size_t rows, size_t cols, float dscale,
                                 RowArgs* a) {
    const size_t n = rows * cols;
    FORGE_TRY(need(sub, n, "norm_bwd row-dot sub"));
    FORGE_TRY(need(dot, rows, "norm_bwd row-dot dot"));
    auto overlap = [](const float* p, size_t pn, const float* q, size_t qn) {
        return pn && qn && p < q + qn && q < p + pn;
    };
    if (overlap(sub.ptr, n, dx.ptr, n))
        return fail(FORGE_EINVAL, "norm_bwd row-dot: sub overlaps dx");
    for (forge_slice m : {x, dy, dx, sub})
        if (overlap(dot.ptr, rows, m.ptr, n))
            return fail(FORGE_EINVAL, "norm_bwd row-dot: dot overlaps a matrix operand");
    a->dsub = sub.ptr;
    a->dot = dot.ptr;
    a->dscale = dscale;
    return FORGE_OK;
}

static forge_status layer_norm_bwd_sgd_impl(forge_runtime* rt, forge_stream* s, forge_slice x,
                                            forge_slice dy, forge_slice gamma, forge_slice beta,
                                            forge_slice dx, forge_slice dgamma, forge_slice dbeta,
                                            size_t rows, size_t cols, float eps, float lr,
                                            const forge_slice* sub, forge_slice dot,
                                            float dscale) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(x, rows * cols, "layer_norm_bwd x"));
    FORGE_TRY(need(dy, rows * cols, "layer_norm_bwd dy"));
    FORGE_TRY(need(dx, rows * cols, "layer_norm_bwd dx"));
    FORGE_TRY(need_opt(gamma, cols, "layer_norm_bwd gamma"));
    FORGE_TRY(need_opt(beta, cols, "layer_norm_bwd beta"));
    FORGE_TRY(need_opt(dgamma, cols, "layer_norm_bwd dgamma"));
    FORGE_TRY(need_opt(dbeta, cols, "layer_norm_bwd dbeta"));
    RowArgs a{x.ptr, dx.ptr, dy.ptr, gamma.ptr, nullptr, nullptr, nullptr, (int)rows, (int)cols, eps, 1.0f};
    if (sub) FORGE_TRY(row_dot_args(x, dy, dx, *sub, dot, rows, cols, dscale, &a));
    NormSgd sgd;
    sgd.gamma = gamma.ptr;
    sgd.beta = beta.ptr;
    sgd.lr = lr;
    return row_launch(rt, s, "layer_norm_bwd", a, dgamma.ptr, dbeta.ptr, nullptr, 0, sgd);
}

extern "C" forge_status forge_layer_norm_bwd_sgd(forge_runtime* rt, forge_stream* s,
                                                 forge_slice x, forge_slice dy,
                                                 forge_slice gamma, forge_slice beta,
                                                 forge_slice dx, forge_slice dgamma,
                                                 forge_slice dbeta, size_t rows, size_t cols,
                                                 float eps, float lr) {
    return layer_norm_bwd_sgd_impl(rt, s, x, dy, gamma, beta, dx, dgamma, dbeta, rows, cols, eps,
                                   lr, nullptr, forge_slice{nullptr, 0}, 1.0f);
}

extern "C" forge_status forge_layer_norm_bwd_sgd_dot(forge_runtime* rt, forge_stream* s,
                                                     forge_slice x, forge_slice dy,
                                                     forge_slice gamma, forge_slice beta,
                                                     forge_slice dx, forge_slice dgamma,
                                                     forge_slice dbeta, forge_slice sub,
                                                     forge_slice dot, size_t rows, size_t cols,
                                                     float eps, float lr, float dot_scale) {
    return layer_norm_bwd_sgd_impl(rt, s, x, dy, gamma, beta, dx, dgamma, dbeta, rows, cols, eps,
                                   lr, &sub, dot, dot_scale);
}

extern "C" forge_status forge_layer_norm_bwd_noalloc(forge_runtime* rt, forge_stream* s,
                                                     forge_slice x, forge_slice dy,
                                                     forge_slice gamma, forge_slice dx,
                                                     forge_slice dgamma, forge_slice dbeta,
                                                     size_t rows, size_t cols, float eps) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (!rt->noalloc_scratch)
        return fail(FORGE_EHIP, "no-allocation scratch unavailable: hipGetSymbolAddress: %s",
                    hipGetErrorString(rt->noalloc_status));
    return layer_norm_bwd_impl(rt, s, x, dy, gamma, dx, dgamma, dbeta, rows, cols, eps,
                               rt->noalloc_scratch, FORGE_NOALLOC_SCRATCH_FLOATS);
}

extern "C" forge_status forge_rms_norm_rows_out(forge_runtime* rt, forge_stream* s,
                                                forge_slice x, forge_slice y, forge_slice gamma,
                                                size_t rows, size_t cols, float eps) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(x, rows * cols, "rms_norm x"));
    FORGE_TRY(need(y, rows * cols, "rms_norm y"));
    FORGE_TRY(check_out_of_place(x, y, rows * cols, "rms_norm"));
    FORGE_TRY(need_opt(gamma, cols, "rms_norm gamma"));
    RowArgs a{x.ptr, y.ptr, nullptr, gamma.ptr, nullptr, nullptr, nullptr, (int)rows, (int)cols, eps, 1.0f};
    return row_launch(rt, s, "rms_norm", a, nullptr, nullptr);
}

extern "C" forge_status forge_rms_norm_rows(forge_runtime* rt, forge_stream* s, forge_slice x,
                                            forge_slice gamma, size_t rows, size_t cols,
                                            float eps) {
    return forge_rms_norm_rows_out(rt, s, x, x, gamma, rows, cols, eps);
}

extern "C" forge_status forge_rms_norm_bwd(forge_runtime* rt, forge_stream* s, forge_slice x,
                                           forge_slice dy, forge_slice gamma, forge_slice dx,
                                           forge_slice dgamma, size_t rows, size_t cols,
                                           float eps) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(x, rows * cols, "rms_norm_bwd x"));
    FORGE_TRY(need(dy, rows * cols, "rms_norm_bwd dy"));
    FORGE_TRY(need(dx, rows * cols, "rms_norm_bwd dx"));
    FORGE_TRY(need_opt(gamma, cols, "rms_norm_bwd gamma"));
    FORGE_TRY(need_opt(dgamma, cols, "rms_norm_bwd dgamma"));
    RowArgs a{x.ptr, dx.ptr, dy.ptr, gamma.ptr, nullptr, nullptr, nullptr, (int)rows, (int)cols, eps, 1.0f};
    return row_launch(rt, s, "rms_norm_bwd", a, dgamma.ptr, nullptr);
}

static forge_status rms_norm_bwd_sgd_impl(forge_runtime* rt, forge_stream* s, forge_slice x,
                                          forge_slice dy, forge_slice gamma, forge_slice dx,
                                          forge_slice dgamma, size_t rows, size_t cols, float eps,
                                          float lr, const forge_slice* sub, forge_slice dot,
                                          float dscale) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(x, rows * cols, "rms_norm_bwd x"));
    FORGE_TRY(need(dy, rows * cols, "rms_norm_bwd dy"));
    FORGE_TRY(need(dx, rows * cols, "rms_norm_bwd dx"));
    FORGE_TRY(need_opt(gamma, cols, "rms_norm_bwd gamma"));
    FORGE_TRY(need_opt(dgamma, cols, "rms_norm_bwd dgamma"));
    RowArgs a{x.ptr, dx.ptr, dy.ptr, gamma.ptr, nullptr, nullptr, nullptr, (int)rows, (int)cols, eps, 1.0f};
    if (sub) FORGE_TRY(row_dot_args(x, dy, dx, *sub, dot, rows, cols, dscale, &a));
    NormSgd sgd;
    sgd.gamma = gamma.ptr;
    sgd.lr = lr;
    return row_launch(rt, s, "rms_norm_bwd", a, dgamma.ptr, nullptr, nullptr, 0, sgd);
}

extern "C" forge_status forge_rms_norm_bwd_sgd(forge_runtime* rt, forge_stream* s, forge_slice x,
                                               forge_slice dy, forge_slice gamma, forge_slice dx,
                                               forge_slice dgamma, size_t rows, size_t cols,
                                               float eps, float lr) {
    return rms_norm_bwd_sgd_impl(rt, s, x, dy, gamma, dx, dgamma, rows, cols, eps, lr, nullptr,
                                 forge_slice{nullptr, 0}, 1.0f);
}

extern "C" forge_status forge_rms_norm_bwd_sgd_dot(forge_runtime* rt, forge_stream* s,
                                                   forge_slice x, forge_slice dy,
                                                   forge_slice gamma, forge_slice dx,
                                                   forge_slice dgamma, forge_slice sub,
                                                   forge_slice dot, size_t rows, size_t cols,
                                                   float eps, float lr, float dot_scale) {
    return rms_norm_bwd_sgd_impl(rt, s, x, dy, gamma, dx, dgamma, rows, cols, eps, lr, &sub, dot,
                                 dot_scale);
}

extern "C" forge_status forge_binary(forge_runtime* rt, forge_stream* s, forge_slice l,
                                     forge_slice r, forge_slice o, size_t n, forge_binary_op op) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    const char* nm = binop_name(op);
    if (!nm) return fail(FORGE_EINVAL, "unknown binary op %d", (int)op);
    FORGE_TRY(need(l, n, "binary l"));
    FORGE_TRY(need(r, n, "binary r"));
    FORGE_TRY(need(o, n, "binary o"));
    if (n == 0) return FORGE_OK;
    bool vec = aligned16(l.ptr) && aligned16(r.ptr) && aligned16(o.ptr);
    char name[64];
    snprintf(name, sizeof name, "forge_binary_%s_%s", nm, vec ? "v" : "s");
    long long nn = (long long)n;
    unsigned g = vec ? stream_grid(nn / 4 + 1) : grid_for(nn, EW_THREADS, 8192);
    return launch_args(rt, s, name, dim3(g), dim3(EW_THREADS), 0, (const float*)l.ptr,
                       (const float*)r.ptr, o.ptr, nn);
}

extern "C" forge_status forge_binary_assign(forge_runtime* rt, forge_stream* s, forge_slice t,
                                            forge_slice r, size_t n, forge_binary_op op) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    const char* nm = binop_name(op);
    if (!nm) return fail(FORGE_EINVAL, "unknown binary op %d", (int)op);
    FORGE_TRY(need(t, n, "binary_assign t"));
    FORGE_TRY(need(r, n, "binary_assign r"));
    if (n == 0) return FORGE_OK;
    bool vec = aligned16(t.ptr) && aligned16(r.ptr);
    char name[64];
    snprintf(name, sizeof name, "forge_binary_assign_%s_%s", nm, vec ? "v" : "s");
    long long nn = (long long)n;
    unsigned g = vec ? stream_grid(nn / 4 + 1) : grid_for(nn, EW_THREADS, 8192);
    return launch_args(rt, s, name, dim3(g), dim3(EW_THREADS), 0, t.ptr, (const float*)r.ptr, nn);
}

extern "C" forge_status forge_sgd_update(forge_runtime* rt, forge_stream* s, forge_slice param,
                                         forge_slice grad, size_t n, float lr) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(need(param, n, "sgd_update param"));
    FORGE_TRY(need(grad, n, "sgd_update grad"));
    if (n == 0) return FORGE_OK;
    bool vec = aligned16(param.ptr) && aligned16(grad.ptr);
    long long nn = (long long)n;
    unsigned g = vec ? stream_grid(nn / 4 + 1) : grid_for(nn, EW_THREADS, 8192);
    return launch_args(rt, s, vec ? "forge_sgd_v" : "forge_sgd_s", dim3(g), dim3(EW_THREADS), 0,
                       param.ptr, (const float*)grad.ptr, nn, lr);
}

extern "C" forge_status forge_binary_assign_by_rows(forge_runtime* rt, forge_stream* s,
                                                    forge_slice m, forge_slice row, size_t rows,
                                                    size_t cols, forge_binary_op op) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    const char* nm = binop_name(op);
    if (!nm) return fail(FORGE_EINVAL, "unknown binary op %d", (int)op);
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(m, rows * cols, "by_rows m"));
    FORGE_TRY(need(row, cols, "by_rows row"));
    if (rows == 0 || cols == 0) return FORGE_OK;
    bool vec = aligned16(m.ptr) && aligned16(row.ptr) && cols % 4 == 0;
    char name[64];
    snprintf(name, sizeof name, "forge_by_rows_%s_%s", nm, vec ? "v" : "s");
    size_t lanes = vec ? cols / 4 : cols;
    unsigned gx = (unsigned)((lanes + EW_THREADS - 1) / EW_THREADS);
    // One row per y index up to the grid's y limit (65535), so a lane
    // moves one float4 as in the streaming kernels; taller matrices loop.
    // At [65536,1024] this took 94 us against 4096 workgroups walking 16
    // rows each.
    unsigned gy = (unsigned)std::min<size_t>(rows, 65535u);
    int r = (int)rows, c = (int)cols;
    return launch_args(rt, s, name, dim3(gx, gy), dim3(EW_THREADS), 0, m.ptr,
                       (const float*)row.ptr, r, c);
}

extern "C" forge_status forge_map(forge_runtime* rt, forge_stream* s, forge_slice x, size_t n,
                                  forge_map_op op, float p0) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    const char* nm = map_name(op);
    if (!nm) return fail(FORGE_EINVAL, "unknown map op %d", (int)op);
    FORGE_TRY(need(x, n, "map x"));
    if (n == 0) return FORGE_OK;
    bool vec = aligned16(x.ptr);
    char name[64];
    snprintf(name, sizeof name, "forge_map_%s_%s", nm, vec ? "v" : "s");
    long long nn = (long long)n;
    unsigned g = vec ? stream_grid(nn / 4 + 1) : grid_for(nn, EW_THREADS, 8192);
    return launch_args(rt, s, name, dim3(g), dim3(EW_THREADS), 0, x.ptr, nn, p0);
}

extern "C" forge_status forge_sum_rows(forge_runtime* rt, forge_stream* s, forge_slice m,
                                       forge_slice out, size_t rows, size_t cols) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(m, rows * cols, "sum_rows m"));
    FORGE_TRY(need(out, rows, "sum_rows out"));
    if (rows == 0) return FORGE_OK;
    bool vec = aligned16(m.ptr) && cols % 4 == 0;
    unsigned g = grid_for((long long)rows, EW_THREADS / 64, 1u << 20);
    int r = (int)rows, c = (int)cols;
    return launch_args(rt, s, vec ? "forge_sum_rows_v" : "forge_sum_rows_s", dim3(g),
                       dim3(EW_THREADS), 0, (const float*)m.ptr, out.ptr, r, c);
}

extern "C" forge_status forge_sum_cols(forge_runtime* rt, forge_stream* s, forge_slice m,
                                       forge_slice out, size_t rows, size_t cols) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(m, rows * cols, "sum_cols m"));
    FORGE_TRY(need(out, cols, "sum_cols out"));
    float* scratch = nullptr;
    size_t need_ws = sum_cols_scratch(rows, cols);
    if (need_ws) FORGE_TRY(workspace(rt, s, need_ws, &scratch));
    return sum_cols_impl(rt, s, m.ptr, ColSumOut{out.ptr, nullptr, 0.0f}, rows, cols, scratch);
}

extern "C" forge_status forge_sum_cols_sgd(forge_runtime* rt, forge_stream* s, forge_slice m,
                                           size_t rows, size_t cols, forge_slice out,
                                           forge_slice param, float lr) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(m, rows * cols, "sum_cols_sgd m"));
    FORGE_TRY(need_opt(out, cols, "sum_cols_sgd out"));
    FORGE_TRY(need_opt(param, cols, "sum_cols_sgd param"));
    if (rows == 0) {
        // Sums of no rows are zero; the step leaves the parameter as it is.
        if (out.ptr) return forge_fill(rt, s, forge_slice{out.ptr, cols}, 0.0f);
        return FORGE_OK;
    }
    float* scratch = nullptr;
    size_t need_ws = sum_cols_scratch(rows, cols);
    if (need_ws) FORGE_TRY(workspace(rt, s, need_ws, &scratch));
    return sum_cols_impl(rt, s, m.ptr, ColSumOut{out.ptr, param.ptr, lr}, rows, cols, scratch);
}

namespace {
// Full reduction of x [n] into out[0]: per-workgroup partials of `kernel`
// (with "_v" appended when x is 16-byte aligned: RED_UNROLL float4 per lane
// per step), then one workgroup of `final_kernel` over the partials.  args0
// is the functor's scalar for map_sum kernels (has_p0).
forge_status reduce_launch(forge_runtime* rt, forge_stream* s, forge_slice x, size_t n,
                           forge_slice out, const char* kernel, const char* final_kernel,
                           bool has_p0, float p0) {
    FORGE_TRY(need(x, n, "reduce x"));
    FORGE_TRY(need(out, 1, "reduce out"));
    const bool vec = aligned16(x.ptr);
    char name[64], fin[64];
    snprintf(name, sizeof name, "%s%s", kernel, vec ? "_v" : "");
    snprintf(fin, sizeof fin, "%s_v", final_kernel);
    long long nn = (long long)n;
    // VEC: RED_UNROLL (4) float4 per lane in flight; scalar: 4 floats per lane.
    const unsigned g = grid_for(vec ? (nn + 3) / 4 : nn, EW_THREADS * 4, 1024);
    auto run = [&](const char* k, unsigned grid, const float* src, long long cnt, float* dst) {
        if (has_p0) return launch_args(rt, s, k, dim3(grid), dim3(EW_THREADS), 0, src, cnt, p0, dst);
        return launch_args(rt, s, k, dim3(grid), dim3(EW_THREADS), 0, src, cnt, dst);
    };
    if (g == 1) return run(name, 1, (const float*)x.ptr, nn, out.ptr);
    float* ws;
    FORGE_TRY(workspace(rt, s, g, &ws));
    FORGE_TRY(run(name, g, (const float*)x.ptr, nn, ws));
    // The partials (aligned workspace) fold with the plain sum or max.
    long long gn = g;
    return launch_args(rt, s, fin, dim3(1), dim3(EW_THREADS), 0, (const float*)ws, gn, out.ptr);
}

forge_status reduce_impl(forge_runtime* rt, forge_stream* s, forge_slice x, size_t n,
                         forge_slice out, bool is_max) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    const char* name = is_max ? "forge_reduce_max" : "forge_reduce_sum";
    return reduce_launch(rt, s, x, n, out, name, name, false, 0.0f);
}
}  // namespace

extern "C" forge_status forge_map_sum(forge_runtime* rt, forge_stream* s, forge_slice x,
                                      size_t n, forge_map_op op, float p0, forge_slice out) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    const char* nm = map_name(op);
    if (!nm) return fail(FORGE_EINVAL, "unknown map op %d", (int)op);
    char name[64];
    snprintf(name, sizeof name, "forge_map_sum_%s", nm);
    return reduce_launch(rt, s, x, n, out, name, "forge_reduce_sum", true, p0);
}

extern "C" forge_status forge_reduce_sum(forge_runtime* rt, forge_stream* s, forge_slice x,
                                         size_t n, forge_slice out) {
    return reduce_impl(rt, s, x, n, out, false);
}

extern "C" forge_status forge_reduce_max(forge_runtime* rt, forge_stream* s, forge_slice x,
                                         size_t n, forge_slice out) {
    return reduce_impl(rt, s, x, n, out, true);
}

extern "C" forge_status forge_softmax_rows_bwd_scaled(forge_runtime* rt, forge_stream* s,
                                                      forge_slice p, forge_slice g,
                                                      forge_slice dx, size_t rows, size_t cols,
                                                      float scale) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    FORGE_TRY(need(p, rows * cols, "softmax_bwd p"));
    FORGE_TRY(need(g, rows * cols, "softmax_bwd g"));
    FORGE_TRY(need(dx, rows * cols, "softmax_bwd dx"));
    RowArgs a{p.ptr, dx.ptr, g.ptr, nullptr, nullptr, nullptr, nullptr, (int)rows, (int)cols, 0.f,
              scale};
    return row_launch(rt, s, "softmax_bwd", a, nullptr, nullptr);
}

extern "C" forge_status forge_activation_backward(forge_runtime* rt, forge_stream* s,
                                                  forge_slice dy, forge_slice z, forge_slice g,
                                                  size_t n, forge_activation act) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    if (act < FORGE_ACT_IDENTITY || act > FORGE_ACT_SILU)
        return fail(FORGE_EINVAL, "unknown activation %d", (int)act);
    FORGE_TRY(need(dy, n, "activation_backward dy"));
    FORGE_TRY(need(z, n, "activation_backward z"));
    FORGE_TRY(need(g, n, "activation_backward g"));
    if (n == 0) return FORGE_OK;
    bool vec = aligned16(dy.ptr) && aligned16(z.ptr) && aligned16(g.ptr);
    long long nn = (long long)n;
    int a = (int)act;
    unsigned grid = vec ? stream_grid(nn / 4 + 1) : grid_for(nn, EW_THREADS, 8192);
    return launch_args(rt, s, vec ? "forge_act_backward_v" : "forge_act_backward_s", dim3(grid),
                       dim3(EW_THREADS), 0, (const float*)dy.ptr, (const float*)z.ptr, g.ptr, nn,
                       a);
}

extern "C" forge_status forge_fill_random(forge_runtime* rt, forge_stream* s, forge_slice x,
                                          size_t n, uint32_t seed) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(need(x, n, "fill_random x"));
    if (n == 0) return FORGE_OK;
    long long nn = (long long)n;
    unsigned sd = seed;
    return launch_args(rt, s, "forge_fill_random", dim3(grid_for(nn, EW_THREADS, 8192)),
                       dim3(EW_THREADS), 0, x.ptr, nn, sd);
}

// Mismatch count of l and r over n elements into out[0] (T: float or u32),
// by the kernels named count and count_final: per-workgroup u32 partials in
// the stream's workspace, summed by one final workgroup.
template <typename T>
static forge_status compare_into(forge_runtime* rt, forge_stream* s, forge_slice l, forge_slice r,
                                 size_t n, T* out, const char* count, const char* count_final) {
    long long nn = (long long)n;
    unsigned g = grid_for(nn, EW_THREADS * 4, 1024);
    if (g == 1)
        return launch_args(rt, s, count, dim3(1), dim3(EW_THREADS), 0, (const float*)l.ptr,
                           (const float*)r.ptr, nn, (unsigned*)nullptr, out);
    float* ws;
    FORGE_TRY(workspace(rt, s, g, &ws));
    unsigned* part = reinterpret_cast<unsigned*>(ws);
    FORGE_TRY(launch_args(rt, s, count, dim3(g), dim3(EW_THREADS), 0, (const float*)l.ptr,
                          (const float*)r.ptr, nn, part, out));
    int gn = (int)g;
    return launch_args(rt, s, count_final, dim3(1), dim3(EW_THREADS), 0, (const unsigned*)part, gn,
                       out);
}

extern "C" forge_status forge_compare(forge_runtime* rt, forge_stream* s, forge_slice l,
                                      forge_slice r, size_t n, forge_slice out) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(need(l, n, "compare l"));
    FORGE_TRY(need(r, n, "compare r"));
    FORGE_TRY(need(out, 1, "compare out"));
    return compare_into(rt, s, l, r, n, out.ptr, "forge_count_neq", "forge_count_final");
}

extern "C" forge_status forge_compare_u32(forge_runtime* rt, forge_stream* s, forge_slice l,
                                          forge_slice r, size_t n, forge_slice_u32 out) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(need(l, n, "compare l"));
    FORGE_TRY(need(r, n, "compare r"));
    FORGE_TRY(need(out, 1, "compare out"));
    return compare_into(rt, s, l, r, n, reinterpret_cast<unsigned*>(out.ptr),
                        "forge_count_neq_u32", "forge_count_final_u32");
}

extern "C" forge_status forge_fill_seq(forge_runtime* rt, forge_stream* s, forge_slice x, size_t n,
                                       int ascending) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(need(x, n, "fill_seq x"));
    if (n == 0) return FORGE_OK;
    long long nn = (long long)n;
    int asc = ascending ? 1 : 0;
    return launch_args(rt, s, "forge_fill_seq", dim3(grid_for(nn, EW_THREADS, 8192)),
                       dim3(EW_THREADS), 0, x.ptr, nn, asc);
}

extern "C" forge_status forge_causal_mask_rows(forge_runtime* rt, forge_stream* s,
                                               forge_slice m, size_t rows, size_t cols,
                                               size_t first_row) {
    if (!rt) return fail(FORGE_EINVAL, "runtime is null");
    FORGE_TRY(check_rows(rows, cols));
    if (!fits_int(first_row) || !fits_int(first_row + rows))
        return fail(FORGE_EINVAL, "first_row + rows exceeds 2^31-1");
    FORGE_TRY(need(m, rows * cols, "causal_mask m"));
    if (rows == 0 || cols == 0) return FORGE_OK;
    unsigned gx = (unsigned)std::min<size_t>((cols + EW_THREADS - 1) / EW_THREADS, 64);
    unsigned gy = (unsigned)std::min<size_t>(rows, 65535);
    int r = (int)rows, c = (int)cols, f = (int)first_row;
    return launch_args(rt, s, "forge_causal_mask", dim3(gx, gy), dim3(EW_THREADS), 0, m.ptr, r, c,
                       f);
}

extern "C" forge_status forge_causal_mask(forge_runtime* rt, forge_stream* s, forge_slice m,
                                          size_t rows, size_t cols) {
    return forge_causal_mask_rows(rt, s, m, rows, cols, 0);
}
