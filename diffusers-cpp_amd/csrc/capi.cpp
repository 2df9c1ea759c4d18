// capi.cpp -- library-level C-ABI: thread-local error text, device
// properties, the backend handle (device + stream), device buffers and
// host<->device tensor transfer.  Stand-ins for the reference's RAII wrappers
// over ggml_backend_dev_t / ggml_backend_t / buffers (src/ggml/Device.hpp,
// Backend.hpp, Buffer.hpp) and ggml_backend_tensor_set/get
// (src/ggml/ExecutionRuntime.cpp:150-156, 302-313).
#include <hip/hip_runtime.h>

#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "capi_util.hpp"
#include "dit_hip.h"
#include "kernels.hpp"

namespace dit {
namespace {
thread_local std::string g_last_error;
std::mutex g_cu_mutex;
std::vector<int> g_cu_counts;
}  // namespace

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_last_error = buf;
    return code;
}

int check_launch(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail(DT_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
    return DT_OK;
}

int cu_count() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return 256;
    std::lock_guard<std::mutex> lock(g_cu_mutex);
    if ((int)g_cu_counts.size() <= dev) g_cu_counts.resize(dev + 1, 0);
    if (g_cu_counts[dev] == 0) {
        int n = 0;
        if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0)
            n = 256;
        g_cu_counts[dev] = n;
    }
    return g_cu_counts[dev];
}

}  // namespace dit

struct dt_backend {
    int device;
    hipStream_t stream;
    void* scratch;
    size_t scratch_bytes;
    float* rope_table;  // (cos, sin) of positions [0, kBackendRopePositions), built on the device
    int rope_axis_dim;
    float rope_base;
    bool own_stream;    // created by dt_graph_capture
    uint64_t generation;  // bumped whenever scratch or rope_table move
};

struct dt_graph_exec {
    hipGraphExec_t exec;
    uint64_t generation;  // the backend's generation at capture
};

extern "C" const char* dt_last_error(void) { return dit::g_last_error.c_str(); }

extern "C" const char* dt_version(void) { return "dit_hip 0.1 (gfx950)"; }

#define DT_HIP(call, what)                                                              \
    do {                                                                                \
        hipError_t e_ = (call);                                                         \
        if (e_ != hipSuccess) return dit::fail(DT_ERR_HIP, "%s: %s", what, hipGetErrorString(e_)); \
    } while (0)

extern "C" int dt_backend_init(int32_t device_ordinal, dt_backend** out) {
    DT_REQUIRE(out != nullptr, "dt_backend_init: null out");
    int n = 0;
    DT_HIP(hipGetDeviceCount(&n), "dt_backend_init");
    DT_REQUIRE(device_ordinal >= 0 && device_ordinal < n, "dt_backend_init: device %d of %d",
               device_ordinal, n);
    DT_HIP(hipSetDevice(device_ordinal), "dt_backend_init");
    void* noalloc = nullptr;  // dt_groupnorm_silu_noalloc's device scratch, resolved for this device now
    const int rc = dit::noalloc_scratch(&noalloc);
    if (rc) return rc;
    auto* be = new dt_backend{device_ordinal, nullptr, nullptr, 0, nullptr, 0, 0.f, false, 0};
    *out = be;
    return DT_OK;
}

extern "C" int dt_backend_free(dt_backend* be) {
    if (!be) return DT_OK;
    if (be->scratch || be->rope_table) {
        (void)hipSetDevice(be->device);
        (void)hipStreamSynchronize(be->stream);
        if (be->scratch) (void)hipFree(be->scratch);
        if (be->rope_table) (void)hipFree(be->rope_table);
    }
    if (be->own_stream) {
        (void)hipStreamSynchronize(be->stream);
        (void)hipStreamDestroy(be->stream);
    }
    delete be;
    return DT_OK;
}

extern "C" int dt_backend_set_stream(dt_backend* be, dt_stream_t stream) {
    DT_REQUIRE(be != nullptr, "dt_backend_set_stream: null backend");
    if (be->own_stream && be->stream != (hipStream_t)stream) {
        DT_HIP(hipSetDevice(be->device), "dt_backend_set_stream");
        DT_HIP(hipStreamSynchronize(be->stream), "dt_backend_set_stream");
        DT_HIP(hipStreamDestroy(be->stream), "dt_backend_set_stream");
        be->own_stream = false;
    }
    be->stream = (hipStream_t)stream;
    return DT_OK;
}

extern "C" int dt_backend_synchronize(dt_backend* be) {
    DT_REQUIRE(be != nullptr, "dt_backend_synchronize: null backend");
    DT_HIP(hipSetDevice(be->device), "dt_backend_synchronize");
    DT_HIP(hipStreamSynchronize(be->stream), "dt_backend_synchronize");
    return DT_OK;
}

extern "C" int dt_buffer_alloc(dt_backend* be, size_t bytes, void** out) {
    DT_REQUIRE(be != nullptr && out != nullptr, "dt_buffer_alloc: null argument");
    DT_HIP(hipSetDevice(be->device), "dt_buffer_alloc");
    void* p = nullptr;
    const hipError_t e = hipMalloc(&p, bytes ? bytes : 1);
    if (e != hipSuccess) return dit::fail(DT_ERR_OOM, "dt_buffer_alloc(%zu): %s", bytes, hipGetErrorString(e));
    *out = p;
    return DT_OK;
}

extern "C" int dt_buffer_free(dt_backend* be, void* ptr) {
    DT_REQUIRE(be != nullptr, "dt_buffer_free: null backend");
    if (!ptr) return DT_OK;
    DT_HIP(hipSetDevice(be->device), "dt_buffer_free");
    DT_HIP(hipFree(ptr), "dt_buffer_free");
    return DT_OK;
}

// Bytes of a contiguous tensor (ggml_nbytes): whole blocks for block types.
// False for negative sizes, unknown types, or a count that overflows int64.
static bool tensor_bytes(const dt_tensor* t, size_t* out) {
    for (int i = 0; i < 4; ++i)
        if (t->ne[i] < 0) return false;
    int64_t n = 1;
    for (int i = 1; i < 4; ++i)
        if (__builtin_mul_overflow(n, t->ne[i], &n)) return false;
    int64_t row = 0;
    const int es = dit::elem_size(t->type);
    if (es) {
        if (__builtin_mul_overflow(t->ne[0], (int64_t)es, &row)) return false;
    } else if (t->type == DT_TYPE_Q8_0) {
        row = (t->ne[0] / 32 + (t->ne[0] % 32 != 0)) * 34;
    } else if (t->type == DT_TYPE_Q4_K) {
        row = (t->ne[0] / 256 + (t->ne[0] % 256 != 0)) * 144;
    } else if (t->type == DT_TYPE_Q8_0_SPLIT) {
        int64_t nk = 0, per = 0, planes = 0, total = 0;
        if (__builtin_mul_overflow(t->ne[0], t->ne[1], &nk) || nk > (1ll << 60) ||
            __builtin_mul_overflow(t->ne[2], t->ne[3], &planes))
            return false;
        per = dt_q8_0_split_bytes(t->ne[1], t->ne[0]);
        if (__builtin_mul_overflow(per, planes, &total)) return false;
        *out = (size_t)total;
        return true;
    } else if (t->type == DT_TYPE_CONV2D_PACKED) {
        if (t->ne[0] > 16 || t->ne[2] > (1 << 20) || t->ne[3] > (1 << 20)) return false;
        *out = dt_conv2d_packed_bytes(t->ne[3], t->ne[2], t->ne[0]);
        return t->ne[1] == t->ne[0] && *out > 0;
    } else {
        return false;
    }
    int64_t bytes = 0;
    if (__builtin_mul_overflow(row, n, &bytes)) return false;
    *out = (size_t)bytes;
    return true;
}

static bool contiguous(const dt_tensor* t) {
    const int es = dit::elem_size(t->type);
    if (es == 0) return true;  // block types: caller addresses raw bytes
    int64_t expect = es;
    for (int i = 0; i < 4; ++i) {
        if (t->ne[i] > 1 && t->nb[i] != (size_t)expect) return false;
        if (i < 3 && __builtin_mul_overflow(expect, t->ne[i], &expect)) return false;
    }
    return true;
}

extern "C" int dt_tensor_set(const dt_tensor* t, const void* host, size_t offset, size_t n,
                             dt_stream_t stream) {
    DT_REQUIRE(t && t->data && (host || n == 0), "dt_tensor_set: null argument");
    DT_REQUIRE(contiguous(t), "dt_tensor_set: tensor is not contiguous");
    size_t total = 0;
    DT_REQUIRE(tensor_bytes(t, &total), "dt_tensor_set: tensor type %d / shape not supported", t->type);
    DT_REQUIRE(offset <= total && n <= total - offset,
               "dt_tensor_set: %zu bytes at offset %zu exceed the tensor's %zu bytes", n, offset, total);
    DT_HIP(hipMemcpyAsync((char*)t->data + offset, host, n, hipMemcpyHostToDevice, (hipStream_t)stream),
           "dt_tensor_set");
    DT_HIP(hipStreamSynchronize((hipStream_t)stream), "dt_tensor_set");
    return DT_OK;
}

extern "C" int dt_tensor_get(const dt_tensor* t, void* host, size_t offset, size_t n,
                             dt_stream_t stream) {
    DT_REQUIRE(t && t->data && (host || n == 0), "dt_tensor_get: null argument");
    DT_REQUIRE(contiguous(t), "dt_tensor_get: tensor is not contiguous");
    size_t total = 0;
    DT_REQUIRE(tensor_bytes(t, &total), "dt_tensor_get: tensor type %d / shape not supported", t->type);
    DT_REQUIRE(offset <= total && n <= total - offset,
               "dt_tensor_get: %zu bytes at offset %zu exceed the tensor's %zu bytes", n, offset, total);
    DT_HIP(hipMemcpyAsync(host, (const char*)t->data + offset, n, hipMemcpyDeviceToHost, (hipStream_t)stream),
           "dt_tensor_get");
    DT_HIP(hipStreamSynchronize((hipStream_t)stream), "dt_tensor_get");
    return DT_OK;
}

namespace dit {

hipStream_t backend_stream(dt_backend* be) { return be ? be->stream : nullptr; }

int backend_device(dt_backend* be) { return be ? be->device : 0; }

int backend_rope_table(dt_backend* be, int axis_dim, float freq_base, const float** out) {
    DT_REQUIRE(be != nullptr && out != nullptr, "backend_rope_table: null argument");
    if (!be->rope_table || be->rope_axis_dim != axis_dim || be->rope_base != freq_base) {
        if (be->rope_table) {
            DT_HIP(hipStreamSynchronize(be->stream), "backend_rope_table");
            DT_HIP(hipFree(be->rope_table), "backend_rope_table");
            be->rope_table = nullptr;
        }
        const size_t bytes = (size_t)kBackendRopePositions * axis_dim * sizeof(float);
        const hipError_t e = hipMalloc(&be->rope_table, bytes);
        if (e != hipSuccess) return fail(DT_ERR_OOM, "backend_rope_table(%zu): %s", bytes, hipGetErrorString(e));
        ++be->generation;
        int rc = rope_table_device(be->rope_table, kBackendRopePositions, axis_dim, freq_base, be->stream);
        if (rc) return rc;
        // Built once; later graphs may run on another stream.
        DT_HIP(hipStreamSynchronize(be->stream), "backend_rope_table");
        be->rope_axis_dim = axis_dim;
        be->rope_base = freq_base;
    }
    *out = be->rope_table;
    return DT_OK;
}

int backend_scratch(dt_backend* be, size_t bytes, void** out) {
    DT_REQUIRE(be != nullptr && out != nullptr, "backend_scratch: null argument");
    if (bytes > be->scratch_bytes) {
        if (be->scratch) {
            // The old buffer may still be read by queued kernels.
            DT_HIP(hipStreamSynchronize(be->stream), "backend_scratch");
            DT_HIP(hipFree(be->scratch), "backend_scratch");
            be->scratch = nullptr;
            be->scratch_bytes = 0;
        }
        ++be->generation;
        const hipError_t e = hipMalloc(&be->scratch, bytes);
        if (e != hipSuccess) return fail(DT_ERR_OOM, "backend_scratch(%zu): %s", bytes, hipGetErrorString(e));
        be->scratch_bytes = bytes;
    }
    *out = be->scratch;
    return DT_OK;
}

}  // namespace dit

extern "C" int dt_graph_capture(dt_backend* be, dt_tensor** nodes, int32_t n_nodes, dt_graph_exec** out) {
    return dt_graph_capture_ex(be, nodes, n_nodes, 0, out);
}

extern "C" int dt_graph_capture_ex(dt_backend* be, dt_tensor** nodes, int32_t n_nodes, uint32_t flags,
                                   dt_graph_exec** out) {
    DT_REQUIRE(be != nullptr && out != nullptr && n_nodes >= 0 && (nodes || n_nodes == 0),
               "dt_graph_capture: bad arguments");
    DT_HIP(hipSetDevice(be->device), "dt_graph_capture");
    if (be->stream == nullptr) {  // the legacy NULL stream cannot be captured
        hipStream_t s = nullptr;
        DT_HIP(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "dt_graph_capture");
        be->stream = s;
        be->own_stream = true;
    }
    DT_HIP(hipStreamSynchronize(be->stream), "dt_graph_capture");
    DT_HIP(hipStreamBeginCapture(be->stream, hipStreamCaptureModeThreadLocal), "dt_graph_capture");
    const uint64_t gen = be->generation;
    const int rc = dt_graph_compute_ex(be, nodes, n_nodes, flags);
    hipGraph_t graph = nullptr;
    const hipError_t e = hipStreamEndCapture(be->stream, &graph);
    if (rc) {
        if (graph) (void)hipGraphDestroy(graph);
        return rc;
    }
    if (e != hipSuccess || !graph)
        return dit::fail(DT_ERR_HIP, "dt_graph_capture: %s (run dt_graph_compute once before capturing)",
                         hipGetErrorString(e));
    hipGraphExec_t exec = nullptr;
    const hipError_t ei = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    (void)hipGraphDestroy(graph);
    if (ei != hipSuccess) return dit::fail(DT_ERR_HIP, "dt_graph_capture: instantiate: %s", hipGetErrorString(ei));
    if (be->generation != gen) {  // the capture itself moved the scratch or the table
        (void)hipGraphExecDestroy(exec);
        return dit::fail(DT_ERR_INVALID_ARG,
                         "dt_graph_capture: the backend's scratch or RoPE table was (re)allocated during capture; "
                         "run dt_graph_compute once before capturing");
    }
    *out = new dt_graph_exec{exec, gen};
    return DT_OK;
}

extern "C" int dt_graph_exec_launch(dt_backend* be, dt_graph_exec* exec) {
    DT_REQUIRE(be != nullptr && exec != nullptr, "dt_graph_exec_launch: null argument");
    DT_REQUIRE(exec->generation == be->generation,
               "dt_graph_exec_launch: the backend's scratch or RoPE table moved since this graph was captured; "
               "capture it again");
    DT_HIP(hipGraphLaunch(exec->exec, be->stream), "dt_graph_exec_launch");
    return DT_OK;
}

extern "C" int dt_graph_exec_free(dt_graph_exec* exec) {
    if (!exec) return DT_OK;
    (void)hipGraphExecDestroy(exec->exec);
    delete exec;
    return DT_OK;
}
