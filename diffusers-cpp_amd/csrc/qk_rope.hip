// qk_rope.hip -- fused per-head RMSNorm(q,k) * w + multi-axis RoPE (NORMAL
// mode, adjacent pairs), the node chain RMSNorm::forward (RMS_NORM + MUL)
// and Flux2PosEmbed::forward (4x ROPE on 32-wide views + 3x CONCAT) emit per
// q and per k (Flux2Attention.hpp:93-122, Flux2ParallelSelfAttention.hpp:
// 52-101, Flux2PosEmbed.hpp:29-108).
//
// Fast path (head_dim 128, axis_dim % 8 == 0): a head is one 16-lane DPP row,
// each lane owns 8 consecutive dims (one 16-byte bf16 load, two for fp32) =
// 4 rotation pairs of a single axis, and a row walks 8 heads of one token.
// The sum of squares is a 4-step DPP row reduction.  cos/sin come from a table built on the host with ggml's
// fp32 angle recurrence, so angles match the CPU op exactly; the table is a
// few tens of KB and stays L2-resident.  q and k go in one launch
// (blockIdx.y selects the tensor); the per-lane norm weights stay in VGPRs.
#include <math.h>

#include <utility>

#include "capi_util.hpp"
#include "common.hpp"
#include "kernels.hpp"
#include "rope_angles.hpp"
#include "swiglu_body.hpp"

namespace dit {
namespace {

struct QkHalf {
    const void* x;
    void* y;
    const float* w;
};

struct QkShape {
    int64_t in_ts, in_hs, out_ts, out_hs;
    RopeAxisPos pos;
    int tokens, heads, head_dim, axis_dim, n_axes, n_pos;
    float eps, theta_scale;
};

// Position pointer and token stride of one axis, chosen with an unrolled
// select so the kernel-argument arrays are never indexed dynamically.
__device__ __forceinline__ void axis_pos(const QkShape& sh, int axis, const int32_t*& p,
                                         int64_t& stride) {
    p = sh.pos.ptr[0];
    stride = sh.pos.stride[0];
#pragma unroll
    for (int a = 1; a < kMaxRopeAxes; ++a) {
        if (axis == a) {
            p = sh.pos.ptr[a];
            stride = sh.pos.stride[a];
        }
    }
}

template <typename T>
__device__ __forceinline__ void load8(const T* p, float* v);
template <>
__device__ __forceinline__ void load8<bf16>(const bf16* p, float* v) { Io<bf16>::load(p, v); }
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* v) {
    Io<float>::load(p, v);
    Io<float>::load(p + 4, v + 4);
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float* v);
template <>
__device__ __forceinline__ void store8<bf16>(bf16* p, const float* v) { Io<bf16>::store(p, v); }
template <>
__device__ __forceinline__ void store8<float>(float* p, const float* v) {
    Io<float>::store(p, v);
    Io<float>::store(p + 4, v + 4);
}

// A work item is one token and up to 4*HPG of its heads: a wave's four
// 16-lane DPP rows take heads h0 + row + 4*i (i < HPG), so each load/store
// instruction covers four consecutive heads = 1 KB of contiguous bf16.  Wave
// w of the W waves of a tensor takes items w, w + W, ... (at most ITER), and
// issues the next item's position and head loads before the current item's
// reduction and rotation, so the loads of every resident wave stay in flight
// while it computes (one item per wave left HBM idle while all resident
// waves computed at once: 23.0 -> 22.2 us for q and k of [4608, 24, 128]).
// The position goes out before the heads: loads retire in issue order, so
// the dependent cos/sin lookup can start while the head loads are still in
// flight.  The lane's 8 norm weights are loaded once per wave.
template <typename T>
struct QkRaw {
    static constexpr int NV = 8 / Io<T>::EPV;  // 16-byte vectors per 8 elements
    uint4 r[NV];
};

template <typename T, int HPG, int NT, int ITER>
__device__ __forceinline__ void qk_rope128_body(const QkHalf& a, const QkShape& sh, const float* __restrict__ table,
                                                int chunks, int block, int W) {
    if (a.x == nullptr) return;
    const int w = (int)((block * NT + threadIdx.x) / kWave);
    if (w >= W) return;  // whole waves leave together
    constexpr int NV = QkRaw<T>::NV, EPV = Io<T>::EPV;
    const int64_t total = (int64_t)sh.tokens * chunks;
    const int lane16 = threadIdx.x & 15;
    const int row = (threadIdx.x & (kWave - 1)) >> 4;
    const int d0 = lane16 * 8;
    const int axis = d0 / sh.axis_dim;
    const int i0 = d0 - axis * sh.axis_dim;
    const T* __restrict__ xb = (const T*)a.x + d0;
    T* __restrict__ yb = (T*)a.y + d0;
    const int32_t* pax;
    int64_t pst;
    axis_pos(sh, axis, pax, pst);

    QkRaw<T> cur[HPG], nxt[HPG];
    int tc = 0, hc = 0, pc = 0, tn = 0, hn = 0, pn = 0;
    // items < tokens * chunks < 2^31 (qk_fast), so an item index fits an int
    auto issue = [&](int j, QkRaw<T>* raw, int& t, int& h0, int& p) {
        t = j / chunks;
        h0 = (j - t * chunks) * 4 * HPG + row;
        p = pax[(int64_t)t * pst];
#pragma unroll
        for (int hh = 0; hh < HPG; ++hh) {
            const int h = h0 + 4 * hh;
#pragma unroll
            for (int u = 0; u < NV; ++u)
                raw[hh].r[u] = h < sh.heads ? ld_stream(xb + (int64_t)t * sh.in_ts + (int64_t)h * sh.in_hs + u * EPV)
                                            : make_uint4(0, 0, 0, 0);
        }
    };
    issue(w, cur, tc, hc, pc);
    float cs[8];
    rope_angles<4>(pc, i0, table, sh.n_pos, sh.axis_dim, sh.theta_scale, cs);
    float wt[8];
#pragma unroll
    for (int e = 0; e < 8; e += 4) {  // shared by every head: default (cached) policy
        const float4 t4 = *reinterpret_cast<const float4*>(a.w + d0 + e);
        wt[e] = t4.x; wt[e + 1] = t4.y; wt[e + 2] = t4.z; wt[e + 3] = t4.w;
    }
    // mean of squares over the 128 dims: the division by 128 is exact, so a
    // multiply by 1/128 gives the quotient's bits
    constexpr float kInvHeadDim = 1.0f / 128.0f;

#pragma unroll
    for (int kk = 0; kk < ITER; ++kk) {
        const int64_t j = w + (int64_t)kk * W;
        if (j >= total) break;
        const bool more = kk + 1 < ITER && j + W < total;
        if (more) issue((int)(j + W), nxt, tn, hn, pn);
#pragma unroll
        for (int hh = 0; hh < HPG; ++hh) {
            const int h = hc + 4 * hh;
            if (h < sh.heads) {  // uniform across the 16 lanes of a DPP row
                float v[8];
#pragma unroll
                for (int u = 0; u < NV; ++u) Io<T>::unpack(cur[hh].r[u], v + u * EPV);
                float ss = 0.f;
#pragma unroll
                for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
                ss = row16_sum(ss);
                const float r = 1.0f / sqrtf(ss * kInvHeadDim + sh.eps);
                float o[8];
#pragma unroll
                for (int qd = 0; qd < 4; ++qd) {
                    const float x0 = mul_rn(mul_rn(v[2 * qd], r), wt[2 * qd]);
                    const float x1 = mul_rn(mul_rn(v[2 * qd + 1], r), wt[2 * qd + 1]);
                    const float c = cs[2 * qd], sn = cs[2 * qd + 1];
                    o[2 * qd] = sub_rn(mul_rn(x0, c), mul_rn(x1, sn));
                    o[2 * qd + 1] = add_rn(mul_rn(x0, sn), mul_rn(x1, c));
                }
                store8<T>(yb + (int64_t)tc * sh.out_ts + (int64_t)h * sh.out_hs, o);
            }
        }
        if (more) {
            rope_angles<4>(pn, i0, table, sh.n_pos, sh.axis_dim, sh.theta_scale, cs);
#pragma unroll
            for (int hh = 0; hh < HPG; ++hh) cur[hh] = nxt[hh];
            tc = tn;
            hc = hn;
        }
    }
}

template <typename T, int HPG, int ITER>
__global__ __launch_bounds__(256) void qk_rope128_kernel(QkHalf q, QkHalf k, QkShape sh,
                                                         const float* __restrict__ table, int chunks, int W) {
    qk_rope128_body<T, HPG, 256, ITER>(blockIdx.y == 0 ? q : k, sh, table, chunks, blockIdx.x, W);
}

constexpr int kQkSwigluThreads = 512;  // the SwiGLU body's best workgroup

// QK-RMSNorm+RoPE of q and k and the SwiGLU of the same block in one launch
// (Flux2ParallelSelfAttention.hpp:55-93: all three read the outputs of the
// block's input projections): blocks [0, qk_blocks) take q, the next
// qk_blocks k (when k is given: n_qk = 2 qk_blocks, else qk_blocks), the
// rest stream the SwiGLU.  The bodies are the standalone kernels', so the
// results are bit-identical to separate launches.
template <typename T, int HPG, int ITER>
__global__ __launch_bounds__(kQkSwigluThreads) void qk_swiglu_kernel(QkHalf q, QkHalf k, QkShape sh,
                                                                     const float* __restrict__ table, int chunks,
                                                                     int W, int qk_blocks, int n_qk, SwigluArgs sw) {
    const int b = blockIdx.x;
    if (b < n_qk)
        qk_rope128_body<T, HPG, kQkSwigluThreads, ITER>(b < qk_blocks ? q : k, sh, table, chunks,
                                                        b < qk_blocks ? b : b - qk_blocks, W);
    else
        swiglu_body<T, kQkSwigluThreads>(sw, b - n_qk);
}

// Any head_dim / axis_dim (even) / stride: one thread per (token, head).
template <typename T>
__global__ __launch_bounds__(256) void qk_rope_generic_kernel(QkHalf q, QkHalf k, QkShape sh,
                                                              const float* __restrict__ table) {
    const QkHalf a = blockIdx.y == 0 ? q : k;
    if (a.x == nullptr) return;
    const int64_t n_groups = (int64_t)sh.tokens * sh.heads;
    const int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= n_groups) return;
    const int64_t t = g / sh.heads, h = g % sh.heads;
    const T* xr = (const T*)a.x + t * sh.in_ts + h * sh.in_hs;
    T* yr = (T*)a.y + t * sh.out_ts + h * sh.out_hs;
    float ss = 0.f;
    for (int d = 0; d < sh.head_dim; ++d) {
        const float v = Io<T>::get(xr + d);
        ss += v * v;
    }
    const float r = 1.0f / sqrtf(ss / (float)sh.head_dim + sh.eps);
    // Pairs are read before either element is written, so y may alias x.
    for (int d = 0; d < sh.head_dim; d += 2) {
        const int axis = d / sh.axis_dim, i0 = d - axis * sh.axis_dim;
        const int32_t* pax;
        int64_t pst;
        axis_pos(sh, axis, pax, pst);
        const int p = pax[t * pst];
        float cs[2];
        if (table != nullptr && p >= 0 && p < sh.n_pos) {
            cs[0] = table[(int64_t)p * sh.axis_dim + i0];
            cs[1] = table[(int64_t)p * sh.axis_dim + i0 + 1];
        } else {
            rope_angles<1>(p, i0, nullptr, 0, sh.axis_dim, sh.theta_scale, cs);
        }
        const float x0 = mul_rn(mul_rn(Io<T>::get(xr + d), r), a.w[d]);
        const float x1 = mul_rn(mul_rn(Io<T>::get(xr + d + 1), r), a.w[d + 1]);
        Io<T>::put(yr + d, sub_rn(mul_rn(x0, cs[0]), mul_rn(x1, cs[1])));
        Io<T>::put(yr + d + 1, add_rn(mul_rn(x0, cs[1]), mul_rn(x1, cs[0])));
    }
}

constexpr int kHPG = 3;  // 12 heads per item: best of HPG in {1, 2, 3, 6} on [4608, 24, 128]
// Items per wave of the standalone launch: 3 keeps every wave of
// [4608, 24, 128] resident at once (6 per SIMD); 2 leaves a second round, 4
// and 8 too few waves (q and k: 22.2 us against 23.0 / 23.9 / 23.7 / 30.5 us
// for 1 / 2 / 4 / 8).  The fused QK+SwiGLU launch takes one item per wave:
// the deeper pipeline's registers (81 against 58 VGPRs) cost its SwiGLU
// blocks occupancy (59.9 us at 1, 61.3 at 2, 67.6 at 3; 62.1-64.4 us for the
// previous single-item body at 71 VGPRs).
constexpr int kQkIter = 3;
constexpr int kQkSwigluIter = 1;

// Waves per tensor for `items` work items at `iter` items per wave.
int64_t qk_waves(int64_t items, int iter) { return (items + iter - 1) / iter; }

template <typename T>
bool qk_fast(const QkHalf& q, const QkHalf& k, const QkShape& sh, const float* table) {
    constexpr int EPV = Io<T>::EPV;
    bool fast = sh.head_dim == 128 && sh.axis_dim % 8 == 0 && sh.in_ts % EPV == 0 &&
                sh.in_hs % EPV == 0 && sh.out_ts % EPV == 0 && sh.out_hs % EPV == 0 &&
                (table == nullptr || aligned16(table));
    const int64_t max_in = (int64_t)(sh.tokens - 1) * sh.in_ts + (int64_t)(sh.heads - 1) * sh.in_hs + sh.head_dim;
    const int64_t max_out = (int64_t)(sh.tokens - 1) * sh.out_ts + (int64_t)(sh.heads - 1) * sh.out_hs + sh.head_dim;
    fast = fast && max_in < (1ll << 31) && max_out < (1ll << 31) &&
           (int64_t)sh.tokens * sh.heads < (1ll << 31);
    for (const QkHalf* h : {&q, &k})
        if (h->x) fast = fast && aligned16(h->x) && aligned16(h->y) && aligned16(h->w);
    return fast;
}

template <typename T>
int run(QkHalf q, QkHalf k, const QkShape& sh, const float* table, hipStream_t st) {
    const bool fast = qk_fast<T>(q, k, sh, table);
    const int ny = k.x ? 2 : 1;
    if (fast) {
        constexpr int HPG = kHPG;
        const int chunks = (sh.heads + 4 * HPG - 1) / (4 * HPG);
        const int64_t waves = qk_waves((int64_t)sh.tokens * chunks, kQkIter);
        const int64_t blocks = (waves + 3) / 4;
        hipLaunchKernelGGL((qk_rope128_kernel<T, HPG, kQkIter>), dim3((unsigned)blocks, ny), dim3(256), 0, st,
                           q, k, sh, table, chunks, (int)waves);
    } else {
        const int64_t groups = (int64_t)sh.tokens * sh.heads;
        const int64_t blocks = (groups + 255) / 256;
        DT_REQUIRE(blocks < (1ll << 31), "dt_qk_rmsnorm_rope: too many heads");
        hipLaunchKernelGGL((qk_rope_generic_kernel<T>), dim3((unsigned)blocks, ny), dim3(256), 0,
                           st, q, k, sh, table);
    }
    return check_launch("dt_qk_rmsnorm_rope");
}

}  // namespace

int qk_prepare(const void* q, const void* k, void* q_out, void* k_out, const float* wq, const float* wk,
               int64_t tokens, int64_t heads, int64_t head_dim, int64_t in_ts, int64_t in_hs, int64_t out_ts,
               int64_t out_hs, float eps, const RopeAxisPos& pos, int n_axes, int axis_dim, float freq_base,
               const float* table, int n_pos, int32_t io, QkHalf* hq_out, QkHalf* hk_out, QkShape* sh_out);

int qk_launch(const void* q, const void* k, void* q_out, void* k_out, const float* wq,
              const float* wk, int64_t tokens, int64_t heads, int64_t head_dim, int64_t in_ts,
              int64_t in_hs, int64_t out_ts, int64_t out_hs, float eps, const RopeAxisPos& pos,
              int n_axes, int axis_dim, float freq_base, const float* table, int n_pos, int32_t io,
              hipStream_t st) {
    QkHalf hq, hk;
    QkShape sh;
    const int rc = qk_prepare(q, k, q_out, k_out, wq, wk, tokens, heads, head_dim, in_ts, in_hs, out_ts, out_hs,
                              eps, pos, n_axes, axis_dim, freq_base, table, n_pos, io, &hq, &hk, &sh);
    if (rc) return rc;
    if (tokens == 0 || (!q && !k)) return DT_OK;
    if (io == DT_TYPE_F32) return run<float>(hq, hk, sh, table, st);
    return run<bf16>(hq, hk, sh, table, st);
}

template <typename T>
int run_qk_swiglu(const QkHalf& hq, const QkHalf& hk, const QkShape& sh, const float* table, const void* g,
                  int64_t gs, const void* u, int64_t us, void* y, int64_t ys, int64_t rows, int64_t cols,
                  hipStream_t st) {
    constexpr int EPV = Io<T>::EPV;
    const int64_t nvec = cols / EPV, total = rows * nvec;
    const bool sw_vec = cols % EPV == 0 && gs % EPV == 0 && us % EPV == 0 && ys % EPV == 0 && aligned16(g) &&
                        aligned16(u) && aligned16(y) && total < (1ll << 31);
    if (!sw_vec || !hq.x || sh.tokens == 0 || rows == 0 || !qk_fast<T>(hq, hk, sh, table)) {
        // shapes the combined kernel does not take: the two launches it
        // replaces, each skipped when its part is empty
        if (hq.x && sh.tokens > 0) {
            const int rc = run<T>(hq, hk, sh, table, st);
            if (rc) return rc;
        }
        return dt_swiglu(g, gs, u, us, y, ys, rows, cols, Io<T>::kType, st);
    }
    constexpr int NT = kQkSwigluThreads, WAVES = NT / kWave;
    const int chunks = (sh.heads + 4 * kHPG - 1) / (4 * kHPG);
    const int64_t waves = qk_waves((int64_t)sh.tokens * chunks, kQkSwigluIter);
    const int64_t qk_blocks = (waves + WAVES - 1) / WAVES;
    const int64_t n_qk = (hk.x ? 2 : 1) * qk_blocks;
    const int64_t blocks = n_qk + swiglu_blocks<T, NT>((uint32_t)total);
    DT_REQUIRE(blocks < (1ll << 31), "dt_qk_rmsnorm_rope_swiglu: grid too large");
    const SwigluArgs sw{g, gs, u, us, y, ys, (uint32_t)total, make_fastdiv((uint32_t)(nvec ? nvec : 1))};
    hipLaunchKernelGGL((qk_swiglu_kernel<T, kHPG, kQkSwigluIter>), dim3((unsigned)blocks), dim3(NT), 0, st, hq, hk, sh,
                       table, chunks, (int)waves, (int)qk_blocks, (int)n_qk, sw);
    return check_launch("dt_qk_rmsnorm_rope_swiglu");
}

int qk_swiglu_launch(const void* q, const void* k, void* q_out, void* k_out, const float* wq, const float* wk,
                     int64_t tokens, int64_t heads, int64_t head_dim, int64_t in_ts, int64_t in_hs, int64_t out_ts,
                     int64_t out_hs, float eps, const RopeAxisPos& pos, int n_axes, int axis_dim, float freq_base,
                     const float* table, int n_pos, const void* g, int64_t gs, const void* u, int64_t us, void* y,
                     int64_t ys, int64_t rows, int64_t cols, int32_t io, hipStream_t st) {
    QkHalf hq, hk;
    QkShape sh;
    const int rc = qk_prepare(q, k, q_out, k_out, wq, wk, tokens, heads, head_dim, in_ts, in_hs, out_ts, out_hs,
                              eps, pos, n_axes, axis_dim, freq_base, table, n_pos, io, &hq, &hk, &sh);
    if (rc) return rc;
    DT_REQUIRE(rows >= 0 && cols > 0 && gs >= cols && us >= cols && ys >= cols,
               "dt_qk_rmsnorm_rope_swiglu: bad SwiGLU shape");
    DT_REQUIRE(rows == 0 || (g && u && y), "dt_qk_rmsnorm_rope_swiglu: null SwiGLU pointer");
    if (io == DT_TYPE_F32) return run_qk_swiglu<float>(hq, hk, sh, table, g, gs, u, us, y, ys, rows, cols, st);
    return run_qk_swiglu<bf16>(hq, hk, sh, table, g, gs, u, us, y, ys, rows, cols, st);
}

int qk_prepare(const void* q, const void* k, void* q_out, void* k_out, const float* wq, const float* wk,
               int64_t tokens, int64_t heads, int64_t head_dim, int64_t in_ts, int64_t in_hs, int64_t out_ts,
               int64_t out_hs, float eps, const RopeAxisPos& pos, int n_axes, int axis_dim, float freq_base,
               const float* table, int n_pos, int32_t io, QkHalf* hq_out, QkHalf* hk_out, QkShape* sh_out) {
    DT_REQUIRE(is_io_type(io), "dt_qk_rmsnorm_rope: io_type %d unsupported", io);
    DT_REQUIRE(tokens >= 0 && heads > 0 && head_dim > 0 && head_dim % 2 == 0,
               "dt_qk_rmsnorm_rope: bad shape");
    DT_REQUIRE(n_axes > 0 && n_axes <= kMaxRopeAxes && axis_dim > 0 && axis_dim % 2 == 0 &&
                   (int64_t)n_axes * axis_dim == head_dim,
               "dt_qk_rmsnorm_rope: need n_axes <= %d and n_axes*axis_dim (%d*%d) == head_dim %lld",
               kMaxRopeAxes, n_axes, axis_dim, (long long)head_dim);
    DT_REQUIRE(in_hs >= head_dim && out_hs >= head_dim && in_ts >= 0 && out_ts >= 0,
               "dt_qk_rmsnorm_rope: bad strides");
    DT_REQUIRE(tokens < (1ll << 31) && heads < (1ll << 31) && head_dim < (1ll << 31),
               "dt_qk_rmsnorm_rope: shape too large");
    DT_REQUIRE(n_pos >= 0, "dt_qk_rmsnorm_rope: n_pos < 0");
    if (tokens > 0 && (q || k)) {
        for (int a = 0; a < n_axes; ++a)
            DT_REQUIRE(pos.ptr[a] != nullptr, "dt_qk_rmsnorm_rope: null position pointer for axis %d", a);
    }
    // an empty input (no tokens) touches no pointer, so its outputs may be null
    DT_REQUIRE(tokens == 0 || !q || (q_out && wq), "dt_qk_rmsnorm_rope: q given without q_out/wq");
    DT_REQUIRE(tokens == 0 || !k || (k_out && wk), "dt_qk_rmsnorm_rope: k given without k_out/wk");
    QkHalf hq{q, q_out, wq}, hk{k, k_out, wk};
    if (!q) std::swap(hq, hk);  // k alone runs as the first half
    QkShape sh;
    sh.in_ts = in_ts; sh.in_hs = in_hs;
    sh.out_ts = out_ts; sh.out_hs = out_hs;
    sh.pos = pos;
    for (int a = n_axes; a < kMaxRopeAxes; ++a) {
        sh.pos.ptr[a] = pos.ptr[0];
        sh.pos.stride[a] = pos.stride[0];
    }
    sh.tokens = (int)tokens; sh.heads = (int)heads; sh.head_dim = (int)head_dim;
    sh.axis_dim = axis_dim; sh.n_axes = n_axes; sh.n_pos = table ? n_pos : 0;
    sh.eps = eps;
    sh.theta_scale = powf(freq_base, -2.0f / (float)axis_dim);
    *hq_out = hq;
    *hk_out = hk;
    *sh_out = sh;
    return DT_OK;
}

namespace {

// One thread per (position, 8-dim chunk): the chunk's four pairs by the
// device recurrence, exactly as the QK kernels compute them without a table.
__global__ __launch_bounds__(256) void rope_table_device_kernel(float* __restrict__ table, int n_pos, int axis_dim,
                                                                float theta_scale) {
    const int chunks = axis_dim / 8;
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= (int64_t)n_pos * chunks) return;
    const int p = (int)(i / chunks), i0 = (int)(i % chunks) * 8;
    float cs[8];
    rope_angles<4>(p, i0, nullptr, 0, axis_dim, theta_scale, cs);
    float* t = table + (int64_t)p * axis_dim + i0;
    *reinterpret_cast<float4*>(t) = make_float4(cs[0], cs[1], cs[2], cs[3]);
    *reinterpret_cast<float4*>(t + 4) = make_float4(cs[4], cs[5], cs[6], cs[7]);
}

}  // namespace

int rope_table_device(float* table, int n_pos, int axis_dim, float freq_base, hipStream_t st) {
    DT_REQUIRE(table && aligned16(table) && n_pos > 0 && axis_dim > 0 && axis_dim % 8 == 0,
               "rope_table_device: bad arguments");
    const int64_t n = (int64_t)n_pos * (axis_dim / 8);
    hipLaunchKernelGGL(rope_table_device_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, st, table, n_pos,
                       axis_dim, powf(freq_base, -2.0f / (float)axis_dim));
    return check_launch("rope_table_device");
}

}  // namespace dit

extern "C" int dt_rope_table_fill(float* table, int32_t n_pos, int32_t n_dims, float freq_base,
                                  float freq_scale, float attn_factor) {
    DT_REQUIRE(table != nullptr && n_pos >= 0 && n_dims > 0 && n_dims % 2 == 0,
               "dt_rope_table_fill: bad arguments");
    const float theta_scale = powf(freq_base, -2.0f / (float)n_dims);
    for (int32_t p = 0; p < n_pos; ++p) {
        float theta = (float)p;
        float* row = table + (int64_t)p * n_dims;
        for (int32_t i0 = 0; i0 < n_dims; i0 += 2) {
            const float t = freq_scale * theta;
            row[i0] = cosf(t) * attn_factor;
            row[i0 + 1] = sinf(t) * attn_factor;
            theta *= theta_scale;
        }
    }
    return DT_OK;
}

extern "C" int dt_qk_rmsnorm_rope(const void* q, const void* k, void* q_out, void* k_out,
                                  int64_t tokens, int64_t heads, int64_t head_dim,
                                  int64_t in_tok_stride, int64_t in_head_stride,
                                  int64_t out_tok_stride, int64_t out_head_stride,
                                  const float* wq, const float* wk, float eps,
                                  const int32_t* pos, int64_t pos_stride, int32_t n_axes,
                                  int32_t axis_dim, float freq_base, const float* rope_table,
                                  int32_t n_pos, int32_t io_type, dt_stream_t stream) {
    DT_REQUIRE(n_axes > 0 && n_axes <= dit::kMaxRopeAxes, "dt_qk_rmsnorm_rope: n_axes %d", n_axes);
    DT_REQUIRE(pos_stride >= n_axes, "dt_qk_rmsnorm_rope: pos_stride < n_axes");
    dit::RopeAxisPos ap{};
    for (int a = 0; a < n_axes; ++a) {
        ap.ptr[a] = pos ? pos + a : nullptr;
        ap.stride[a] = pos_stride;
    }
    return dit::qk_launch(q, k, q_out, k_out, wq, wk, tokens, heads, head_dim, in_tok_stride,
                          in_head_stride, out_tok_stride, out_head_stride, eps, ap, n_axes,
                          axis_dim, freq_base, rope_table, n_pos, io_type, (hipStream_t)stream);
}

extern "C" int dt_qk_rmsnorm_rope_swiglu(const void* q, const void* k, void* q_out, void* k_out, int64_t tokens,
                                         int64_t heads, int64_t head_dim, int64_t in_tok_stride,
                                         int64_t in_head_stride, int64_t out_tok_stride, int64_t out_head_stride,
                                         const float* wq, const float* wk, float eps, const int32_t* pos,
                                         int64_t pos_stride, int32_t n_axes, int32_t axis_dim, float freq_base,
                                         const float* rope_table, int32_t n_pos, const void* gate,
                                         int64_t gate_stride, const void* up, int64_t up_stride, void* y,
                                         int64_t y_stride, int64_t rows, int64_t inner, int32_t io_type,
                                         dt_stream_t stream) {
    DT_REQUIRE(n_axes > 0 && n_axes <= dit::kMaxRopeAxes, "dt_qk_rmsnorm_rope_swiglu: n_axes %d", n_axes);
    DT_REQUIRE(pos_stride >= n_axes, "dt_qk_rmsnorm_rope_swiglu: pos_stride < n_axes");
    dit::RopeAxisPos ap{};
    for (int a = 0; a < n_axes; ++a) {
        ap.ptr[a] = pos ? pos + a : nullptr;
        ap.stride[a] = pos_stride;
    }
    return dit::qk_swiglu_launch(q, k, q_out, k_out, wq, wk, tokens, heads, head_dim, in_tok_stride, in_head_stride,
                                 out_tok_stride, out_head_stride, eps, ap, n_axes, axis_dim, freq_base, rope_table,
                                 n_pos, gate, gate_stride, up, up_stride, y, y_stride, rows, inner, io_type,
                                 (hipStream_t)stream);
}
