// gn_single_pass.hip -- measurement probe: GroupNorm(G) + per-channel affine
// + SiLU over NCHW in ONE pass over x.  Each workgroup keeps its chunk of a
// group in registers, reduces it to (mean, M2), publishes that record, and
// meets the other workgroups of its group at a per-group barrier in device
// memory; then every workgroup merges the group's records in the same fixed
// order and applies y = silu(fma(x - mean, rstd * w_c, b_c)) to the values it
// still holds.  x is read from HBM once (the library's GroupNorm reads it
// twice, groupnorm.hip), at the price of a device-wide dependency per group.
// It exists to measure that price; no graph or module uses it.
//
// Every workgroup of the grid must be resident at once, or a barrier would
// wait for a workgroup that cannot start: the launcher picks the vectors per
// thread so that the grid fits the device's occupancy and refuses maps that
// do not fit.  Every wait is bounded: a barrier wait that runs past
// `spin_limit` polls sets the error word and the kernel still finishes.
//
// Two forms of the barrier (`form`):
//   0  acquire/release at agent scope: the records are plain stores, made
//      visible by a release fence before the arrival and an acquire fence
//      after the wait (on gfx950 a write-back and an invalidate of the L2);
//   1  every shared word through device-scope relaxed atomics, with a
//      workgroup fence ordering the record stores before the arrival (the
//      form that avoids the L2 maintenance).
// The barrier words of a group are one count and one generation, 128 bytes
// apart from the next group's.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "common.hpp"

namespace {

using namespace dit;

constexpr int kThreads = 256;
constexpr int kSyncStride = 32;  // unsigned words per group's barrier (128 bytes)
constexpr int kMaxRecords = 4096;  // workgroups per group

struct Args {
    const void* x;
    void* y;
    const float* w;
    const float* b;
    int64_t cg, group_len, group_vecs;
    int G, wpg;  // groups per sample; workgroups per group
    float eps;
    int silu, form;
    double2* rec;     // per workgroup: (mean, M2) of its chunk
    unsigned* sync;   // per group: count, generation
    unsigned* err;
    FastDiv hw_vecs;
    unsigned spin_limit;
};

template <typename T, int V>
__global__ __launch_bounds__(kThreads) void gn_single_pass_kernel(Args a) {
    constexpr int EPV = Io<T>::EPV;
    __shared__ double red[kThreads / kWave];
    const int ng = blockIdx.x / a.wpg, wi = blockIdx.x - ng * a.wpg;
    const int n = ng / a.G, g = ng - n * a.G;
    const int64_t off = ((int64_t)n * a.G + g) * a.group_len;
    const T* xg = static_cast<const T*>(a.x) + off;
    T* yg = static_cast<T*>(a.y) + off;
    const int64_t v0 = (int64_t)wi * (V * kThreads);
    const int64_t v1 = v0 + V * kThreads < a.group_vecs ? v0 + V * kThreads : a.group_vecs;

    uint4 raw[V];
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int64_t v = v0 + threadIdx.x + (int64_t)i * kThreads;
        if (v < v1) raw[i] = ld_stream(xg + v * EPV);
    }
    // The chunk's mean, then its M2 around the fp32 mean (the values are in
    // registers), corrected to the fp64 mean.
    double s = 0.0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int64_t v = v0 + threadIdx.x + (int64_t)i * kThreads;
        if (v < v1) {
            float f[EPV];
            Io<T>::unpack(raw[i], f);
            float p = 0.f;
#pragma unroll
            for (int e = 0; e < EPV; ++e) p += f[e];
            s += (double)p;
        }
    }
    const double cnt = (double)((v1 - v0) * EPV);
    const double mw = block_sum_f64(s, red) / cnt;
    const float mwf = (float)mw;
    double q = 0.0;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int64_t v = v0 + threadIdx.x + (int64_t)i * kThreads;
        if (v < v1) {
            float f[EPV];
            Io<T>::unpack(raw[i], f);
            float p = 0.f;
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                const float d = f[e] - mwf;
                p += d * d;
            }
            q += (double)p;
        }
    }
    const double dm = mw - (double)mwf;
    const double m2 = block_sum_f64(q, red) - cnt * dm * dm;

    double2* rec = a.rec + (int64_t)ng * a.wpg;
    if (threadIdx.x == 0) {
        unsigned* count = a.sync + (int64_t)ng * kSyncStride;
        unsigned* gen = count + 1;
        unsigned spins = 0;
        if (a.form == 0) {
            rec[wi] = make_double2(mw, m2);
            __threadfence();
            const unsigned g0 = __hip_atomic_load(gen, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned old = __hip_atomic_fetch_add(count, 1u, __ATOMIC_ACQ_REL, __HIP_MEMORY_SCOPE_AGENT);
            if (old == (unsigned)a.wpg - 1) {
                __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __hip_atomic_fetch_add(gen, 1u, __ATOMIC_RELEASE, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                while (__hip_atomic_load(gen, __ATOMIC_ACQUIRE, __HIP_MEMORY_SCOPE_AGENT) == g0) {
                    __builtin_amdgcn_s_sleep(1);
                    if (++spins > a.spin_limit) {
                        __hip_atomic_fetch_or(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                }
            }
            __threadfence();
        } else {
            __hip_atomic_store(&rec[wi].x, mw, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __hip_atomic_store(&rec[wi].y, m2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            const unsigned g0 = __hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
            const unsigned old = __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (old == (unsigned)a.wpg - 1) {
                __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
                __hip_atomic_fetch_add(gen, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            } else {
                while (__hip_atomic_load(gen, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) == g0) {
                    __builtin_amdgcn_s_sleep(1);
                    if (++spins > a.spin_limit) {
                        __hip_atomic_fetch_or(a.err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                        break;
                    }
                }
            }
        }
    }
    __syncthreads();

    // The group's records merged in a fixed order by every wave: the group
    // mean from the chunk means, then M2 = sum (M2_i + n_i (mean_i - mean)^2).
    const int lane = threadIdx.x & (kWave - 1);
    const double per = (double)V * kThreads * EPV;
    double sm = 0.0;
    for (int i = lane; i < a.wpg; i += kWave) {
        const double mi = __hip_atomic_load(&rec[i].x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const double ni = i == a.wpg - 1 ? (double)a.group_len - per * (a.wpg - 1) : per;
        sm += ni * mi;
    }
    const double mean = wave_sum_f64(sm) / (double)a.group_len;
    double sq = 0.0;
    for (int i = lane; i < a.wpg; i += kWave) {
        const double mi = __hip_atomic_load(&rec[i].x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const double qi = __hip_atomic_load(&rec[i].y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const double ni = i == a.wpg - 1 ? (double)a.group_len - per * (a.wpg - 1) : per;
        sq += qi + ni * (mi - mean) * (mi - mean);
    }
    double var = wave_sum_f64(sq) / (double)a.group_len;
    if (var < 0.0) var = 0.0;
    const float meanf = (float)mean;
    const float rstd = 1.0f / sqrtf((float)var + a.eps);
    const int64_t c0 = (int64_t)g * a.cg;
#pragma unroll
    for (int i = 0; i < V; ++i) {
        const int64_t v = v0 + threadIdx.x + (int64_t)i * kThreads;
        if (v < v1) {
            float f[EPV];
            Io<T>::unpack(raw[i], f);
            const int64_t c = c0 + (int64_t)fdiv((uint32_t)v, a.hw_vecs);
            const float sa = a.w ? rstd * a.w[c] : rstd, bc = a.b ? a.b[c] : 0.0f;
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                const float t = __builtin_fmaf(f[e] - meanf, sa, bc);
                f[e] = a.silu ? silu_fast(t) : t;
            }
            Io<T>::store(yg + v * EPV, f);
        }
    }
}

template <typename T, int V>
int resident_blocks(int cus) {
    int per_cu = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, gn_single_pass_kernel<T, V>, kThreads, 0) != hipSuccess)
        return 0;
    return per_cu * cus;
}

template <typename T, int V>
int try_launch(Args a, int64_t groups, int cus, hipStream_t st) {
    const int64_t per = (int64_t)V * kThreads;
    const int64_t wpg = (a.group_vecs + per - 1) / per;
    if (wpg > kMaxRecords || wpg * groups > resident_blocks<T, V>(cus)) return 0;
    a.wpg = (int)wpg;
    hipLaunchKernelGGL((gn_single_pass_kernel<T, V>), dim3((unsigned)(wpg * groups)), dim3(kThreads), 0, st, a);
    return hipGetLastError() == hipSuccess ? (int)(wpg * groups) : -2;
}

template <typename T>
int launch(Args a, int64_t groups, int cus, hipStream_t st) {
    int r = 0;
    if ((r = try_launch<T, 1>(a, groups, cus, st)) != 0) return r;
    if ((r = try_launch<T, 2>(a, groups, cus, st)) != 0) return r;
    if ((r = try_launch<T, 4>(a, groups, cus, st)) != 0) return r;
    if ((r = try_launch<T, 8>(a, groups, cus, st)) != 0) return r;
    if ((r = try_launch<T, 16>(a, groups, cus, st)) != 0) return r;
    return -1;
}

}  // namespace

// Bytes of workspace for N x C x HW in G groups (barrier words, error word,
// records); it must be zero before the first call and is left reusable.
extern "C" int64_t dt_probe_gn_single_pass_workspace_bytes(int64_t N, int64_t C, int64_t HW, int64_t G) {
    (void)C;
    (void)HW;
    const int64_t groups = N * G;
    return (groups * kSyncStride + 64) * 4 + groups * kMaxRecords * (int64_t)sizeof(double2);
}

// One single-pass GroupNorm(+SiLU) of x [N][C][HW] (io_type 0: fp32, 1: bf16;
// 16-byte aligned rows, HW * C / G a multiple of the 16-byte vector) into y.
// Returns the number of workgroups launched; -1 when the grid cannot be
// resident at once, -2 on a launch error, -3 on bad arguments.  The error
// word (at byte N * G * 128 of the workspace) is non-zero after a call whose
// barrier wait ran out.
extern "C" int dt_probe_gn_single_pass(const void* x, void* y, const float* w, const float* b, int64_t N, int64_t C,
                                       int64_t HW, int64_t G, float eps, int silu, int io_type, int form,
                                       void* workspace, int64_t workspace_bytes, hipStream_t stream) {
    const int epv = io_type == 1 ? 8 : 4;
    if (!x || !y || !workspace || N <= 0 || G <= 0 || C % G != 0 || (C / G * HW) % epv != 0 || HW % epv != 0 ||
        (io_type != 0 && io_type != 1) || (form != 0 && form != 1) ||
        workspace_bytes < dt_probe_gn_single_pass_workspace_bytes(N, C, HW, G))
        return -3;
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess ||
        hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        return -2;
    Args a{};
    a.x = x;
    a.y = y;
    a.w = w;
    a.b = b;
    a.cg = C / G;
    a.group_len = a.cg * HW;
    a.group_vecs = a.group_len / epv;
    a.G = (int)G;
    a.eps = eps;
    a.silu = silu;
    a.form = form;
    const int64_t groups = N * G;
    a.sync = static_cast<unsigned*>(workspace);
    a.err = a.sync + groups * kSyncStride;
    a.rec = reinterpret_cast<double2*>(static_cast<char*>(workspace) + (groups * kSyncStride + 64) * 4);
    a.hw_vecs = make_fastdiv((uint32_t)(HW / epv));
    a.spin_limit = 1u << 22;
    return io_type == 1 ? launch<bf16>(a, groups, cus, stream) : launch<float>(a, groups, cus, stream);
}
