// stream_probe.hip -- the streaming ceiling bench.py sets the fused chain
// beside: trivial-math kernels with a fused launch's exact access shape (the
// same buffers, the same byte counts per stream, 16-byte non-temporal loads
// and stores, 512-thread workgroups, one vector per thread), so the ratio
// chain / probe says how much of the bandwidth this GPU actually gives such
// a stream the kernels reach.  Measurement only: no graph or module uses it.
//
// A launch has up to two segments, like the fused QK+SwiGLU launch (its q/k
// half: 2 streams in, 2 out; its SwiGLU half: 2 in, 1 out).  Segment s reads
// a[i] (and b[i]) and writes y[i] = a ^ b (and z[i] = a + b) for i < n
// 16-byte vectors.
#include <hip/hip_runtime.h>
#include <cstdint>

namespace {

typedef unsigned int v4u __attribute__((ext_vector_type(4)));

struct Segment {
    const v4u* a;
    const v4u* b;  // NULL: one input stream
    v4u* y;
    v4u* z;        // NULL: one output stream
    int64_t n;     // 16-byte vectors per stream
};

constexpr int kThreads = 512;

__global__ __launch_bounds__(kThreads) void stream_probe_kernel(Segment s0, Segment s1, int64_t blocks0) {
    const bool first = blockIdx.x < blocks0;
    const Segment& s = first ? s0 : s1;
    const int64_t i = (first ? (int64_t)blockIdx.x : (int64_t)blockIdx.x - blocks0) * kThreads + threadIdx.x;
    if (i >= s.n) return;
    const v4u va = __builtin_nontemporal_load(s.a + i);
    const v4u vb = s.b ? __builtin_nontemporal_load(s.b + i) : va;
    __builtin_nontemporal_store(va ^ vb, s.y + i);
    if (s.z) __builtin_nontemporal_store(va + vb, s.z + i);
}

bool aligned16(const void* p) { return ((uintptr_t)p & 15) == 0; }

}  // namespace

// Segment k: in[2k], in[2k+1] (may be NULL) -> out[2k], out[2k+1] (may be
// NULL), n[k] vectors of 16 bytes each (n[1] == 0: one segment).  Returns 0,
// or 1 for bad arguments, 2 for a launch error.
extern "C" int dt_stream_probe(const void* const* in, void* const* out, const int64_t* n, hipStream_t stream) {
    Segment s[2];
    for (int k = 0; k < 2; ++k) {
        s[k] = Segment{(const v4u*)in[2 * k], (const v4u*)in[2 * k + 1], (v4u*)out[2 * k], (v4u*)out[2 * k + 1],
                       n[k]};
        if (n[k] < 0 || (n[k] > 0 && (!s[k].a || !s[k].y))) return 1;
        for (const void* p : {(const void*)s[k].a, (const void*)s[k].b, (const void*)s[k].y, (const void*)s[k].z})
            if (p && !aligned16(p)) return 1;
    }
    const int64_t b0 = (n[0] + kThreads - 1) / kThreads, b1 = (n[1] + kThreads - 1) / kThreads;
    if (b0 + b1 == 0) return 0;
    if (b0 + b1 >= (1ll << 31)) return 1;
    hipLaunchKernelGGL(stream_probe_kernel, dim3((unsigned)(b0 + b1)), dim3(kThreads), 0, stream, s[0], s[1], b0);
    return hipGetLastError() == hipSuccess ? 0 : 2;
}
