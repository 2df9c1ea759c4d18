// groupnorm.hip -- GroupNorm(G, eps) + per-channel affine + SiLU over NCHW,
// the NORM -> MUL -> ADD -> SIGMOID -> MUL chain of GroupNorm::forward
// (GroupNorm.cpp:25-108) followed by SiLU::forward (SiLU.hpp:9-13) in the
// VAE decoder (ResnetBlock2D.inl:111-122, 160-171; Decoder.hpp:147-160).
//
// A group is C/G contiguous channels = up to 16.8 M elements, far beyond one
// workgroup, so the reduction is split deterministically:
//   1. stats: each workgroup reduces a fixed chunk of one group to
//      (sum d, sum d^2) with d = x - K (K = the group's first element, a
//      shift that removes cancellation), fp32 over 16-byte vectors and fp64
//      across vectors/lanes, written to its own workspace slot;
//   2. apply: each workgroup issues its chunk's loads, then sums its
//      group's partials in a fixed order (every workgroup of a group gets
//      bit-identical statistics) while those loads are in flight, then
//      streams out y = silu(((x - mean) * rstd) * w_c + b_c).  The partials
//      and the chunk arrive in one memory latency, not two in a row.
// x is read twice (1.5x the algorithmic bytes).  Measured on gfx950: stats
// loads that allocate in the caches, and running the two passes group batch
// by group batch so the re-read could come from the 256 MB last-level cache,
// were both slower than streaming both reads; a single pass holding the whole
// map in registers across the chip (per-group barrier) was no faster on the
// maps that fit, where fixed launch and ramp costs dominate.
//
// The apply math is y = silu((x - mean) * (rstd * w_c) + b_c): one exact
// subtraction and one fma, then x / (1 + 2^(-x log2 e)) by the hardware exp2
// and reciprocal (relative error ~1e-6 against the graph's separately
// rounded NORM, MUL, ADD, SIGMOID, MUL).  The exactly rounded form took
// ~35 VALU instructions per element and made the bf16 passes VALU-bound.
#include <mutex>

#include "capi_util.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace dit {
namespace {

constexpr int kBlock = 256;
constexpr int kVecsPerThread = 4;            // vectors per thread per chunk
constexpr int kChunkVecs = kBlock * kVecsPerThread;

struct GnShape {
    int64_t C, HW, cg, group_len;            // group_len = cg * HW elements
    int64_t group_vecs;                      // group_len / EPV (or group_len when scalar)
    int G, nchunks;
    float eps;
    int apply_silu;
};

template <typename T, bool VEC>
__device__ __forceinline__ int epv_of() {
    return VEC ? Io<T>::EPV : 1;
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kBlock) void gn_stats_kernel(const T* __restrict__ x, GnShape s,
                                                          double* __restrict__ ws) {
    constexpr int EPV = VEC ? Io<T>::EPV : 1;
    __shared__ double red[2 * kBlock / kWave];
    const int ng = blockIdx.y, n = ng / s.G, g = ng - n * s.G;
    const T* xg = x + (int64_t)n * s.C * s.HW + (int64_t)g * s.group_len;
    const float K = Io<T>::get(xg);
    const int64_t v0 = (int64_t)blockIdx.x * kChunkVecs;
    int64_t v1 = v0 + kChunkVecs;
    if (v1 > s.group_vecs) v1 = s.group_vecs;
    double s1 = 0.0, s2 = 0.0;
    // The thread's vectors are all requested before the first is used (kept
    // packed, 4 registers each), so a wave has kVecsPerThread in flight.
    uint4 raw[kVecsPerThread];
    if constexpr (VEC) {
#pragma unroll
        for (int i = 0; i < kVecsPerThread; ++i) {
            const int64_t v = v0 + threadIdx.x + (int64_t)i * kBlock;
            if (v < v1) raw[i] = ld_stream(xg + v * EPV);
        }
    }
#pragma unroll
    for (int i = 0; i < kVecsPerThread; ++i) {
        const int64_t v = v0 + threadIdx.x + (int64_t)i * kBlock;
        if (v >= v1) break;
        float a[EPV];
        if constexpr (VEC) Io<T>::unpack(raw[i], a);
        else a[0] = Io<T>::get(xg + v);
        float p1 = 0.f, p2 = 0.f;
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
            const float d = a[e] - K;
            p1 += d;
            p2 += d * d;
        }
        s1 += (double)p1;
        s2 += (double)p2;
    }
    block_sum2_f64(s1, s2, red);  // one LDS exchange: small maps 2-4% faster
    double* slot = ws + (int64_t)ng * (2 * s.nchunks + 1);
    if (threadIdx.x == 0) {
        slot[1 + 2 * blockIdx.x] = s1;
        slot[2 + 2 * blockIdx.x] = s2;
        if (blockIdx.x == 0) slot[0] = (double)K;
    }
}

// This workgroup's chunk of group (n, g): the thread's vectors are loaded
// (packed; see gn_stats_kernel) by gn_chunk_load, then gn_chunk_finish
// computes y = silu((x - mean) * (rstd * w_c) + b_c) and stores it.
template <typename T, bool VEC, int AV = kVecsPerThread>
__device__ __forceinline__ void gn_chunk_load(const T* x, const GnShape& s, int n, int g, uint4 (&raw)[AV]) {
    constexpr int EPV = VEC ? Io<T>::EPV : 1;
    if constexpr (VEC) {
        const T* xg = x + (int64_t)n * s.C * s.HW + (int64_t)g * s.group_len;
        const int64_t v0 = (int64_t)blockIdx.x * (kBlock * AV);
        const int64_t v1 = v0 + kBlock * AV < s.group_vecs ? v0 + kBlock * AV : s.group_vecs;
#pragma unroll
        for (int i = 0; i < AV; ++i) {
            const int64_t v = v0 + threadIdx.x + (int64_t)i * kBlock;
            if (v < v1) raw[i] = ld_stream(xg + v * EPV);
        }
    }
}

template <typename T, bool VEC, int AV = kVecsPerThread>
__device__ __forceinline__ void gn_chunk_finish(const T* x, const GnShape& s, int n, int g, float mean, float rstd,
                                                const float* __restrict__ w, const float* __restrict__ b, T* y,
                                                FastDiv hw_vecs, const uint4 (&raw)[AV]) {
    constexpr int EPV = VEC ? Io<T>::EPV : 1;
    const int64_t off = (int64_t)n * s.C * s.HW + (int64_t)g * s.group_len;
    const T* xg = x + off;
    T* yg = y + off;
    const int64_t c0 = (int64_t)g * s.cg;
    const int64_t v0 = (int64_t)blockIdx.x * (kBlock * AV);
    int64_t v1 = v0 + kBlock * AV;
    if (v1 > s.group_vecs) v1 = s.group_vecs;
#pragma unroll
    for (int i = 0; i < AV; ++i) {
        const int64_t v = v0 + threadIdx.x + (int64_t)i * kBlock;
        if (v >= v1) break;
        float a[EPV];
        if constexpr (VEC) Io<T>::unpack(raw[i], a);
        else a[0] = Io<T>::get(xg + v);
        const int64_t c = c0 + (int64_t)fdiv((uint32_t)v, hw_vecs);
        const float sa = w ? rstd * w[c] : rstd, bc = b ? b[c] : 0.0f;
#pragma unroll
        for (int e = 0; e < EPV; ++e) {
            const float t = __builtin_fmaf(a[e] - mean, sa, bc);
            a[e] = s.apply_silu ? silu_fast(t) : t;
        }
        if constexpr (VEC) Io<T>::store(yg + v * EPV, a);
        else Io<T>::put(yg + v, a[0]);
    }
}

// Group ng's (mean, rstd) from its stats partials, summed in a fixed order
// (every caller gets bit-identical values).  Up to one partial per lane:
// each wave sums them itself (an xor butterfly, whose every lane ends with
// the same value), so the small maps' apply pass has no LDS round trip or
// barrier before its math; more partials: the whole workgroup, through LDS.
__device__ __forceinline__ void gn_group_stats(const double* __restrict__ ws, const GnShape& s, int ng,
                                               double* red, float* mean, float* rstd) {
    const double* slot = ws + (int64_t)ng * (2 * s.nchunks + 1);
    double s1 = 0.0, s2 = 0.0;
    if (s.nchunks <= kWave) {
        const int lane = threadIdx.x & (kWave - 1);
        if (lane < s.nchunks) {
            s1 = slot[1 + 2 * lane];
            s2 = slot[2 + 2 * lane];
        }
        s1 = wave_sum_f64(s1);
        s2 = wave_sum_f64(s2);
    } else {
        for (int i = threadIdx.x; i < s.nchunks; i += kBlock) {
            s1 += slot[1 + 2 * i];
            s2 += slot[2 + 2 * i];
        }
        s1 = block_sum_f64(s1, red);
        s2 = block_sum_f64(s2, red);
    }
    const double inv_len = 1.0 / (double)s.group_len;
    const double dm = s1 * inv_len;
    double var = s2 * inv_len - dm * dm;
    if (var < 0.0) var = 0.0;
    *mean = (float)(slot[0] + dm);
    *rstd = 1.0f / sqrtf((float)var + s.eps);
}

// AV vectors per thread: the apply pass's own chunking (kBlock * AV
// vectors per workgroup), independent of the statistics pass's chunks,
// whose partials it sums; the output is the same for any AV.
template <typename T, bool VEC, int AV = kVecsPerThread>
__global__ __launch_bounds__(kBlock) void gn_apply_kernel(const T* x, GnShape s,
                                                          const double* __restrict__ ws,
                                                          const float* __restrict__ w,
                                                          const float* __restrict__ b, T* y,
                                                          FastDiv hw_vecs) {
    __shared__ double red[kBlock / kWave];
    const int ng = blockIdx.y, n = ng / s.G, g = ng - n * s.G;
    uint4 raw[AV];
    gn_chunk_load<T, VEC, AV>(x, s, n, g, raw);
    float mean, rstd;
    gn_group_stats(ws, s, ng, red, &mean, &rstd);
    gn_chunk_finish<T, VEC, AV>(x, s, n, g, mean, rstd, w, b, y, hw_vecs, raw);
}

// (mean, rstd) of every group, for a consumer that applies the
// normalisation itself (the 3x3 conv's channel-last copy).
__global__ __launch_bounds__(kBlock) void gn_mean_rstd_kernel(const double* __restrict__ ws, GnShape s,
                                                              float2* __restrict__ mr) {
    __shared__ double red[kBlock / kWave];
    float mean, rstd;
    gn_group_stats(ws, s, blockIdx.x, red, &mean, &rstd);
    if (threadIdx.x == 0) mr[blockIdx.x] = make_float2(mean, rstd);
}

// Statistics from per-tile (mean, M2, count) records, as dt_conv2d_gn writes
// them: one workgroup per (n, g) merges its group's records with Chan's
// pairwise update in fp64 -- each thread a fixed strided subset in order,
// then a fixed-shape tree -- and stores (mean, variance).
__device__ __forceinline__ void chan_merge(double& n, double& m, double& m2, double nb, double mb, double m2b) {
    if (nb == 0.0) return;
    const double t = n + nb, d = mb - m;
    m += d * (nb / t);
    m2 += m2b + d * d * (n * nb / t);
    n = t;
}

__global__ __launch_bounds__(kBlock) void gn_tile_stats_finalize_kernel(const float4* __restrict__ tiles,
                                                                        int n_tiles, double2* __restrict__ out) {
    __shared__ double sn[kBlock], sm[kBlock], s2[kBlock];
    const int ng = blockIdx.x;
    const float4* rec = tiles + (int64_t)ng * n_tiles;
    double n = 0.0, m = 0.0, m2 = 0.0;
    for (int i = threadIdx.x; i < n_tiles; i += kBlock) {
        const float4 r = rec[i];
        chan_merge(n, m, m2, (double)r.z, (double)r.x, (double)r.y);
    }
    sn[threadIdx.x] = n;
    sm[threadIdx.x] = m;
    s2[threadIdx.x] = m2;
    __syncthreads();
    for (int h = kBlock / 2; h > 0; h >>= 1) {
        if ((int)threadIdx.x < h) {
            double a = sn[threadIdx.x], am = sm[threadIdx.x], a2 = s2[threadIdx.x];
            chan_merge(a, am, a2, sn[threadIdx.x + h], sm[threadIdx.x + h], s2[threadIdx.x + h]);
            sn[threadIdx.x] = a;
            sm[threadIdx.x] = am;
            s2[threadIdx.x] = a2;
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) out[ng] = make_double2(sm[0], sn[0] > 0.0 ? s2[0] / sn[0] : 0.0);
}

template <typename T, bool VEC>
__global__ __launch_bounds__(kBlock) void gn_apply_stats_kernel(const T* x, GnShape s,
                                                                const double2* __restrict__ mv,
                                                                const float* __restrict__ w,
                                                                const float* __restrict__ b, T* y,
                                                                FastDiv hw_vecs) {
    const int ng = blockIdx.y, n = ng / s.G, g = ng - n * s.G;
    uint4 raw[kVecsPerThread];
    gn_chunk_load<T, VEC>(x, s, n, g, raw);
    const double2 r = mv[ng];
    const float mean = (float)r.x;
    const float rstd = 1.0f / sqrtf((float)r.y + s.eps);
    gn_chunk_finish<T, VEC>(x, s, n, g, mean, rstd, w, b, y, hw_vecs, raw);
}

int64_t chunks_for(int64_t group_vecs) { return (group_vecs + kChunkVecs - 1) / kChunkVecs; }

template <typename T, bool VEC>
int launch(const void* x, const GnShape& s, int64_t N, const float* w, const float* b, void* y,
           double* ws, hipStream_t st) {
    constexpr int EPV = VEC ? Io<T>::EPV : 1;
    const dim3 grid((unsigned)s.nchunks, (unsigned)(N * s.G));
    hipLaunchKernelGGL((gn_stats_kernel<T, VEC>), grid, dim3(kBlock), 0, st, (const T*)x, s, ws);
    int rc = check_launch("dt_groupnorm_silu(stats)");
    if (rc) return rc;
    const FastDiv hv = make_fastdiv((uint32_t)(s.HW / EPV));
    // Two vectors per thread when four would leave fewer than 2048 apply
    // workgroups (8 per CU on 256 CUs): the bf16 [1, 512, 128, 128] map,
    // 1024 -> 2048 workgroups, the shape of the fastest plain copy of its
    // bytes.  Four above that (every other decoder map measured faster so).
    const int64_t half_chunks = (s.group_vecs + 2 * kBlock - 1) / (2 * kBlock);
    if (VEC && (int64_t)s.nchunks * N * s.G < 2048) {
        const dim3 g2((unsigned)half_chunks, (unsigned)(N * s.G));
        hipLaunchKernelGGL((gn_apply_kernel<T, VEC, 2>), g2, dim3(kBlock), 0, st, (const T*)x, s, ws, w, b, (T*)y, hv);
    } else {
        hipLaunchKernelGGL((gn_apply_kernel<T, VEC>), grid, dim3(kBlock), 0, st, (const T*)x, s, ws, w, b, (T*)y, hv);
    }
    return check_launch("dt_groupnorm_silu(apply)");
}

}  // namespace
}  // namespace dit

static bool gn_vec_ok(int64_t HW, int32_t io_type) {
    const int epv = io_type == DT_TYPE_BF16 ? 8 : 4;
    return HW % epv == 0;
}

extern "C" size_t dt_groupnorm_workspace_bytes(int64_t N, int64_t C, int64_t HW, int64_t groups) {
    if (N <= 0 || C <= 0 || HW <= 0 || groups <= 0 || C % groups != 0) return 0;
    // Sized for the scalar path (one element per "vector"), the larger case.
    const int64_t nchunks = dit::chunks_for(C / groups * HW);
    return (size_t)(N * groups * (2 * nchunks + 1)) * sizeof(double);
}

// Workspace bytes the launch for these pointers needs: the vector path's
// chunk count when x and y take 16-byte vectors, else the scalar path's.
static size_t gn_workspace_needed(const void* x, const void* y, int64_t N, int64_t C, int64_t HW, int64_t groups,
                                  int32_t io_type) {
    const bool vec = gn_vec_ok(HW, io_type) && dit::aligned16(x) && dit::aligned16(y);
    const int epv = vec ? (io_type == DT_TYPE_BF16 ? 8 : 4) : 1;
    const int64_t nchunks = dit::chunks_for(C / groups * HW / epv);
    return (size_t)(N * groups * (2 * nchunks + 1)) * sizeof(double);
}

static int gn_check_shape(const char* what, const void* x, const void* y, int64_t N, int64_t C, int64_t HW,
                          int64_t groups, int32_t io_type) {
    DT_REQUIRE(dit::is_io_type(io_type), "%s: io_type %d unsupported", what, io_type);
    DT_REQUIRE(N >= 0 && C > 0 && HW >= 0 && groups > 0 && C % groups == 0,
               "%s: bad shape N=%lld C=%lld HW=%lld groups=%lld", what, (long long)N, (long long)C,
               (long long)HW, (long long)groups);
    if (N == 0 || HW == 0) return DT_OK;  // empty: the caller returns before touching anything
    DT_REQUIRE(x && y, "%s: null pointer", what);
    DT_REQUIRE(N * groups < 65536, "%s: N*groups must be < 65536", what);
    return DT_OK;
}

static int gn_run(const void* x, int64_t N, int64_t C, int64_t HW, int64_t groups, const float* w, const float* b,
                  float eps, int32_t apply_silu, void* y, void* workspace, int32_t io_type, dt_stream_t stream);

extern "C" int dt_groupnorm_silu(const void* x, int64_t N, int64_t C, int64_t HW, int64_t groups,
                                 const float* w, const float* b, float eps, int32_t apply_silu,
                                 void* y, void* workspace, size_t workspace_bytes, int32_t io_type,
                                 dt_stream_t stream) {
    int rc = gn_check_shape("dt_groupnorm_silu", x, y, N, C, HW, groups, io_type);
    if (rc) return rc;
    if (N == 0 || HW == 0) return DT_OK;
    DT_REQUIRE(workspace, "dt_groupnorm_silu: null workspace");
    DT_REQUIRE(workspace_bytes >= dt_groupnorm_workspace_bytes(N, C, HW, groups),
               "dt_groupnorm_silu: workspace too small (%zu < %zu)", workspace_bytes,
               dt_groupnorm_workspace_bytes(N, C, HW, groups));
    DT_REQUIRE(((uintptr_t)workspace & 7) == 0, "dt_groupnorm_silu: workspace must be 8-byte aligned");
    return gn_run(x, N, C, HW, groups, w, b, eps, apply_silu, y, workspace, io_type, stream);
}

// ---- the variant that allocates nothing ---------------------------------------
//
// Its statistics workspace is this file-scope device array: each device the
// library runs on holds one copy, at its own address, until the process
// ends.  Host code uses the address hipGetSymbolAddress reports for the
// current device (resolved once per device, at dt_backend_init or at the
// first call), never the array's name.  Every call on a device shares that
// device's copy: calls that overlap on one device (other streams) race.
// Nothing in it has to start at zero: each call's statistics pass writes
// every slot its apply pass reads.
static __device__ __align__(256) unsigned char scratch[DT_GROUPNORM_NOALLOC_SCRATCH_BYTES];

namespace dit {

namespace {
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};
}  // namespace

// The current device's address of `scratch`, resolved once per device.
int noalloc_scratch(void** out) {
    int dev = 0;
    const hipError_t e = hipGetDevice(&dev);
    if (e != hipSuccess) return fail(DT_ERR_HIP, "dt_groupnorm_silu_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    DT_REQUIRE(dev >= 0 && dev < kMaxDevices, "dt_groupnorm_silu_noalloc: device %d beyond %d", dev, kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (r != hipSuccess || !p)
            return fail(DT_ERR_HIP, "dt_groupnorm_silu_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                        hipGetErrorString(r));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return DT_OK;
}

}  // namespace dit

extern "C" int dt_groupnorm_silu_noalloc(const void* x, int64_t N, int64_t C, int64_t HW, int64_t groups,
                                         const float* w, const float* b, float eps, int32_t apply_silu, void* y,
                                         int32_t io_type, dt_stream_t stream) {
    int rc = gn_check_shape("dt_groupnorm_silu_noalloc", x, y, N, C, HW, groups, io_type);
    if (rc) return rc;
    if (N == 0 || HW == 0) return DT_OK;
    const size_t need = gn_workspace_needed(x, y, N, C, HW, groups, io_type);
    DT_REQUIRE(need <= (size_t)DT_GROUPNORM_NOALLOC_SCRATCH_BYTES,
               "dt_groupnorm_silu_noalloc: N=%lld C=%lld HW=%lld groups=%lld needs %zu bytes of statistics, "
               "beyond its %zu-byte device scratch (use dt_groupnorm_silu with a workspace)",
               (long long)N, (long long)C, (long long)HW, (long long)groups, need,
               (size_t)DT_GROUPNORM_NOALLOC_SCRATCH_BYTES);
    void* ws = nullptr;
    rc = dit::noalloc_scratch(&ws);
    if (rc) return rc;
    return gn_run(x, N, C, HW, groups, w, b, eps, apply_silu, y, ws, io_type, stream);
}

static int gn_run(const void* x, int64_t N, int64_t C, int64_t HW, int64_t groups, const float* w, const float* b,
                  float eps, int32_t apply_silu, void* y, void* workspace, int32_t io_type, dt_stream_t stream) {
    const bool vec = gn_vec_ok(HW, io_type) && dit::aligned16(x) && dit::aligned16(y);
    const int epv = vec ? (io_type == DT_TYPE_BF16 ? 8 : 4) : 1;
    dit::GnShape s;
    s.C = C;
    s.HW = HW;
    s.cg = C / groups;
    s.group_len = s.cg * HW;
    s.group_vecs = s.group_len / epv;
    s.G = (int)groups;
    s.nchunks = (int)dit::chunks_for(s.group_vecs);
    s.eps = eps;
    s.apply_silu = apply_silu ? 1 : 0;
    DT_REQUIRE(s.group_vecs < (1ll << 31), "dt_groupnorm_silu: group too large");
    hipStream_t st = (hipStream_t)stream;
    double* ws = (double*)workspace;
    if (io_type == DT_TYPE_F32)
        return vec ? dit::launch<float, true>(x, s, N, w, b, y, ws, st)
                   : dit::launch<float, false>(x, s, N, w, b, y, ws, st);
    return vec ? dit::launch<dit::bf16, true>(x, s, N, w, b, y, ws, st)
               : dit::launch<dit::bf16, false>(x, s, N, w, b, y, ws, st);
}

namespace dit {

int gn_mean_rstd(const void* x, int64_t N, int64_t C, int64_t HW, int64_t groups, float eps, void* workspace,
                 float2* mr, int32_t io_type, hipStream_t st) {
    int rc = gn_check_shape("GroupNorm statistics", x, mr, N, C, HW, groups, io_type);
    if (rc) return rc;
    DT_REQUIRE(N > 0 && HW > 0 && workspace && ((uintptr_t)workspace & 7) == 0,
               "GroupNorm statistics: empty input or bad workspace");
    // The vector path exactly when the unfused GroupNorm takes it: its
    // statistics' partial sums depend on it.  That output is 16-byte aligned
    // wherever an allocator places it, so x alone decides.
    const bool vec = gn_vec_ok(HW, io_type) && aligned16(x);
    const int epv = vec ? (io_type == DT_TYPE_BF16 ? 8 : 4) : 1;
    GnShape s;
    s.C = C;
    s.HW = HW;
    s.cg = C / groups;
    s.group_len = s.cg * HW;
    s.group_vecs = s.group_len / epv;
    s.G = (int)groups;
    s.nchunks = (int)chunks_for(s.group_vecs);
    s.eps = eps;
    s.apply_silu = 0;
    DT_REQUIRE(s.group_vecs < (1ll << 31), "GroupNorm statistics: group too large");
    const dim3 grid((unsigned)s.nchunks, (unsigned)(N * s.G));
    double* ws = (double*)workspace;
    if (io_type == DT_TYPE_F32) {
        if (vec) hipLaunchKernelGGL((gn_stats_kernel<float, true>), grid, dim3(kBlock), 0, st, (const float*)x, s, ws);
        else hipLaunchKernelGGL((gn_stats_kernel<float, false>), grid, dim3(kBlock), 0, st, (const float*)x, s, ws);
    } else {
        if (vec) hipLaunchKernelGGL((gn_stats_kernel<bf16, true>), grid, dim3(kBlock), 0, st, (const bf16*)x, s, ws);
        else hipLaunchKernelGGL((gn_stats_kernel<bf16, false>), grid, dim3(kBlock), 0, st, (const bf16*)x, s, ws);
    }
    rc = check_launch("GroupNorm statistics");
    if (rc) return rc;
    hipLaunchKernelGGL(gn_mean_rstd_kernel, dim3((unsigned)(N * groups)), dim3(kBlock), 0, st, ws, s, mr);
    return check_launch("GroupNorm statistics (mean, rstd)");
}

int gn_tile_stats_finalize(const void* stats, int64_t N, int64_t groups, int64_t n_tiles, hipStream_t st) {
    hipLaunchKernelGGL(gn_tile_stats_finalize_kernel, dim3((unsigned)(N * groups)), dim3(kBlock), 0, st,
                       (const float4*)((const char*)stats + gn_tile_stats_head_bytes(N, groups)), (int)n_tiles,
                       (double2*)stats);
    return check_launch("dt_conv2d_gn(stats)");
}

}  // namespace dit

extern "C" int dt_groupnorm_silu_from_stats(const void* x, int64_t N, int64_t C, int64_t HW, int64_t groups,
                                            const void* stats, const float* w, const float* b, float eps,
                                            int32_t apply_silu, void* y, int32_t io_type, dt_stream_t stream) {
    DT_REQUIRE(dit::is_io_type(io_type), "dt_groupnorm_silu_from_stats: io_type %d unsupported", io_type);
    DT_REQUIRE(N > 0 && C > 0 && HW > 0 && groups > 0 && C % groups == 0,
               "dt_groupnorm_silu_from_stats: bad shape");
    DT_REQUIRE(x && y && stats, "dt_groupnorm_silu_from_stats: null pointer");
    DT_REQUIRE(((uintptr_t)stats & 15) == 0, "dt_groupnorm_silu_from_stats: stats must be 16-byte aligned");
    DT_REQUIRE(N * groups < 65536, "dt_groupnorm_silu_from_stats: N*groups must be < 65536");
    const bool vec = gn_vec_ok(HW, io_type) && dit::aligned16(x) && dit::aligned16(y);
    const int epv = vec ? (io_type == DT_TYPE_BF16 ? 8 : 4) : 1;
    dit::GnShape s;
    s.C = C;
    s.HW = HW;
    s.cg = C / groups;
    s.group_len = s.cg * HW;
    s.group_vecs = s.group_len / epv;
    s.G = (int)groups;
    s.nchunks = (int)dit::chunks_for(s.group_vecs);
    s.eps = eps;
    s.apply_silu = apply_silu ? 1 : 0;
    DT_REQUIRE(s.group_vecs < (1ll << 31), "dt_groupnorm_silu_from_stats: group too large");
    const dim3 grid((unsigned)s.nchunks, (unsigned)(N * s.G));
    const dit::FastDiv hv = dit::make_fastdiv((uint32_t)(s.HW / epv));
    hipStream_t st = (hipStream_t)stream;
    const double2* mv = (const double2*)stats;
    using dit::bf16;
    if (io_type == DT_TYPE_F32) {
        if (vec) hipLaunchKernelGGL((dit::gn_apply_stats_kernel<float, true>), grid, dim3(dit::kBlock), 0, st,
                                    (const float*)x, s, mv, w, b, (float*)y, hv);
        else hipLaunchKernelGGL((dit::gn_apply_stats_kernel<float, false>), grid, dim3(dit::kBlock), 0, st,
                                (const float*)x, s, mv, w, b, (float*)y, hv);
    } else {
        if (vec) hipLaunchKernelGGL((dit::gn_apply_stats_kernel<bf16, true>), grid, dim3(dit::kBlock), 0, st,
                                    (const bf16*)x, s, mv, w, b, (bf16*)y, hv);
        else hipLaunchKernelGGL((dit::gn_apply_stats_kernel<bf16, false>), grid, dim3(dit::kBlock), 0, st,
                                (const bf16*)x, s, mv, w, b, (bf16*)y, hv);
    }
    return dit::check_launch("dt_groupnorm_silu_from_stats");
}
