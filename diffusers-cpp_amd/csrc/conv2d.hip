// conv2d.hip -- the VAE decoder's convolutions on MFMA: ggml_conv_2d_direct
// (stride 1, dilation 1, square kernel K in {1, 3}, padding (K-1)/2) plus the
// bias ADD of Conv2d::forward (src/nn/modules/conv/Conv2d.cpp:37-108), NCHW,
// optionally reading the nearest 2x upscale of its input, the
// `upscale(x, 2, NEAREST)` that precedes the conv in Upsample2D::forward
// (Upsample2D.cpp:36-63), so the 4x larger upscaled tensor is never stored.
//
// Implicit GEMM with the weights as the MFMA A operand:
//   C^T[co][p] = sum over (tap, ci) of W[co][tap][ci] * X[ci][pixel p + tap]
// (the operand roles of the Linear GEMM, so each lane ends up holding
// consecutive pixels of one output channel row: coalesced NCHW stores).
//   - Weights are repacked once (dt_conv2d_pack_weights) to bf16
//     [Co pad 128][K*K][Ci pad 32]: 8 consecutive input channels of one
//     (co, tap) are one 16-byte operand.
//   - A workgroup computes 128 output channels x 128 output pixels, a TR x TC
//     rectangle (TC = 128, 64, 32 or 16 by the output width); four waves of
//     64 x 64.  Per chunk of CI input channels it stages the input patch
//     ((TR + K - 1) x (TC + K - 1) pixels, channel-last, bf16) and the weight
//     slice ([128][K*K][CI]) in LDS; each 64-byte channel record is stored
//     16-byte-unit-swizzled (unit u of record r at u ^ ((r >> 1) & 3)) so
//     that 8 consecutive pixels or output channels read distinct banks.
//   - Operands are rounded to bf16 (as the Linear GEMM's); sums are fp32 in
//     MFMA order; the epilogue adds the bias in fp32 and stores fp32 or bf16.
#include <algorithm>

#include "capi_util.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace dit {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kTileCo = 128, kTilePx = 128, kCi = 32;  // channels per LDS chunk
constexpr int kRec = kCi * 2;                           // bytes per staged pixel / weight record

__device__ __forceinline__ int rec_swz(int r) { return (r >> 1) & 3; }

struct ConvArgs {
    const void* x;
    const uint16_t* w;  // packed bf16 [Co_pad][KK][Ci_pad]
    const float* bias;
    void* y;
    int N, Ci, H, W;     // input (before the optional upscale)
    int Co, K, up2;
    int Hs, Ws;          // the convolved image (upscaled or not) = output size
    int Ci_pad, KK;
    int TR, TC, tiles_w; // pixel tile geometry; tiles along the width
    float4* stats;       // GroupNorm tile records [N][G][pixel tiles] (dt_conv2d_gn), or null
    int G, cg;           // groups over Co and channels per group (cg divides 128)
};

template <typename TI>
__device__ __forceinline__ float load_in(const TI* p);
template <>
__device__ __forceinline__ float load_in<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_in<bf16>(const bf16* p) {
    return __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
}

// The value a store of v as T keeps.
template <typename T>
__device__ __forceinline__ float stored_value(float v);
template <>
__device__ __forceinline__ float stored_value<float>(float v) { return v; }
template <>
__device__ __forceinline__ float stored_value<bf16>(float v) { return bf16_lo(pack_bf16x2(v, 0.f)); }

// GroupNorm statistics of one output tile, as the stored (rounded) values:
// per group of cg channels, the tile's mean and M2 = sum (v - mean)^2 over
// its valid pixels (two passes over the values parked in LDS, fp32), written
// as one (mean, M2, count, 0) record.  Every thread of the workgroup calls it.
template <typename T>
__device__ __forceinline__ void conv_group_stats(const ConvArgs& a, const f32x16_t (&acc)[2][2], uint8_t* smem,
                                                 int co0, int oh0, int ow0, int wco, int wpx, int lrow, int g) {
    float* tb = reinterpret_cast<float*>(smem);  // [128 co][128 px]
    float* red = tb + kTileCo * kTilePx;
    const int rows_valid = min(a.TR, a.Hs - oh0), cols_valid = min(a.TC, a.Ws - ow0);
    // The main loop ended with a barrier: LDS is free.
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = wpx + 32 * i + lrow;
        const bool valid = p / a.TC < rows_valid && p % a.TC < cols_valid;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int cl = wco + 32 * j + 8 * (r >> 2) + 4 * g + (r & 3);
                float v = acc[j][i][r];
                if (a.bias && co0 + cl < a.Co) v = add_rn(v, a.bias[co0 + cl]);
                tb[cl * kTilePx + p] = valid ? stored_value<T>(v) : 0.f;
            }
    }
    __syncthreads();
    const int tid = threadIdx.x;
    const int tpg = 256 / (kTileCo / a.cg);  // threads per group (a power of two)
    const int gi = tid / tpg, ti = tid - gi * tpg;
    const float* gv = tb + gi * a.cg * kTilePx;  // the group's rows are contiguous
    const int n_el = a.cg * kTilePx;
    const int vp = rows_valid * cols_valid;
    auto seg_sum = [&](float v) {
        red[tid] = v;
        __syncthreads();
        for (int h = tpg / 2; h > 0; h >>= 1) {
            if (ti < h) red[tid] += red[tid + h];
            __syncthreads();
        }
        const float r = red[gi * tpg];
        __syncthreads();
        return r;
    };
    float s1 = 0.f;
    for (int e = ti; e < n_el; e += tpg) s1 += gv[e];  // invalid pixels hold 0
    const float mean = seg_sum(s1) / (float)(a.cg * vp);
    float s2 = 0.f;
    for (int e = ti; e < n_el; e += tpg) {
        const int p = e & (kTilePx - 1);
        if (p / a.TC < rows_valid && p % a.TC < cols_valid) {
            const float d = gv[e] - mean;
            s2 += d * d;
        }
    }
    const float m2 = seg_sum(s2);
    const int grp = co0 / a.cg + gi;
    if (ti == 0 && grp < a.G)
        a.stats[((int64_t)blockIdx.z * a.G + grp) * gridDim.x + blockIdx.x] =
            make_float4(mean, m2, (float)(a.cg * vp), 0.f);
}

template <typename T, int K, bool STATS>
__global__ __launch_bounds__(256) void conv2d_kernel(const ConvArgs a) {
    constexpr int KK = K * K, PAD = (K - 1) / 2;
    constexpr int W_BYTES = kTileCo * KK * kRec;
    // input patch: up to (TR + K - 1) x (TC + K - 1) pixels; TR x TC = 128
    constexpr int X_MAX = (128 + K - 1) * (1 + K - 1) > (16 + K - 1) * (8 + K - 1)
                              ? (128 + K - 1) * (1 + K - 1) : (16 + K - 1) * (8 + K - 1);
    // With STATS the epilogue reuses LDS for the tile's stored values (64 KB)
    // and a 256-float reduction array.
    constexpr int MAIN_BYTES = W_BYTES + X_MAX * kRec;
    constexpr int STAT_BYTES = kTileCo * kTilePx * 4 + 256 * 4;
    __shared__ __attribute__((aligned(16))) uint8_t smem[STATS && STAT_BYTES > MAIN_BYTES ? STAT_BYTES : MAIN_BYTES];
    uint8_t* Ws_ = smem;
    uint8_t* Xs = smem + W_BYTES;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = blockIdx.z, co0 = blockIdx.y * kTileCo;
    const int th = blockIdx.x / a.tiles_w, tw = blockIdx.x - th * a.tiles_w;
    const int oh0 = th * a.TR, ow0 = tw * a.TC;
    const int PR = a.TR + K - 1, PC = a.TC + K - 1;  // staged patch rows / cols
    const int wco = (wave >> 1) * 64, wpx = (wave & 1) * 64;
    const int lrow = lane & 31, g = lane >> 5;
    const T* x = reinterpret_cast<const T*>(a.x) + (int64_t)n * a.Ci * a.H * a.W;

    f32x16_t acc[2][2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.f;

    // LDS offsets of this lane's B operands: pixel p = wpx + 32 i + lrow of the
    // tile, at patch position (p / TC + kh, p % TC + kw).
    int pbase[2];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = wpx + 32 * i + lrow;
        pbase[i] = (p / a.TC) * PC + (p % a.TC);
    }

    for (int c0 = 0; c0 < a.Ci_pad; c0 += kCi) {
        // Stage the weights: [128 co][KK][32 ci] from the packed tensor.
        const uint16_t* wg = a.w + ((int64_t)co0 * KK) * a.Ci_pad + c0;
        for (int u = tid; u < kTileCo * KK * 4; u += 256) {
            const int rec = u >> 2, part = u & 3;  // rec = co * KK + tap
            const uint4 v = *reinterpret_cast<const uint4*>(wg + (int64_t)rec * a.Ci_pad + part * 8);
            *reinterpret_cast<uint4*>(Ws_ + rec * kRec + ((part ^ rec_swz(rec)) << 4)) = v;
        }
        // Stage the input patch, channel-last: unit (pixel, 8 channels).
        for (int u = tid; u < PR * PC * 4; u += 256) {
            const int part = u / (PR * PC), pix = u - part * PR * PC;
            const int pr = pix / PC, pc = pix - pr * PC;
            const int ih = oh0 + pr - PAD, iw = ow0 + pc - PAD;
            float v[8];
            const bool inside = ih >= 0 && ih < a.Hs && iw >= 0 && iw < a.Ws;
            const int sh = a.up2 ? ih >> 1 : ih, sw = a.up2 ? iw >> 1 : iw;
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const int ci = c0 + part * 8 + e;
                v[e] = inside && ci < a.Ci ? load_in<T>(x + ((int64_t)ci * a.H + sh) * a.W + sw) : 0.f;
            }
            const uint4 packed = make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]),
                                            pack_bf16x2(v[4], v[5]), pack_bf16x2(v[6], v[7]));
            *reinterpret_cast<uint4*>(Xs + pix * kRec + ((part ^ rec_swz(pix)) << 4)) = packed;
        }
        __syncthreads();
#pragma unroll
        for (int tap = 0; tap < KK; ++tap) {
            const int kh = tap / K, kw = tap - kh * K;
#pragma unroll
            for (int kk = 0; kk < 2; ++kk) {
                const int unit = 2 * kk + g;  // 8-channel unit of this lane's k range
                bf16x8_t wf[2], xf[2];
#pragma unroll
                for (int j = 0; j < 2; ++j) {
                    const int rec = (wco + 32 * j + lrow) * KK + tap;
                    wf[j] = *reinterpret_cast<const bf16x8_t*>(Ws_ + rec * kRec + ((unit ^ rec_swz(rec)) << 4));
                }
#pragma unroll
                for (int i = 0; i < 2; ++i) {
                    const int pix = pbase[i] + kh * PC + kw;
                    xf[i] = *reinterpret_cast<const bf16x8_t*>(Xs + pix * kRec + ((unit ^ rec_swz(pix)) << 4));
                }
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int i = 0; i < 2; ++i)
                        acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j], xf[i], acc[j][i], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // Epilogue: lane holds C^T[co][p] for co = wco + 32 j + 8 (r / 4) + 4 g + r % 4,
    // p = wpx + 32 i + lrow.
    T* y = reinterpret_cast<T*>(a.y) + (int64_t)n * a.Co * a.Hs * a.Ws;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int p = wpx + 32 * i + lrow;
        const int oh = oh0 + p / a.TC, ow = ow0 + p % a.TC;
        if (oh >= a.Hs || ow >= a.Ws) continue;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int co = co0 + wco + 32 * j + 8 * (r >> 2) + 4 * g + (r & 3);
                if (co >= a.Co) continue;
                float v = acc[j][i][r];
                if (a.bias) v = add_rn(v, a.bias[co]);
                Io<T>::put(y + ((int64_t)co * a.Hs + oh) * a.Ws + ow, v);
            }
        }
    }
    if constexpr (STATS) conv_group_stats<T>(a, acc, smem, co0, oh0, ow0, wco, wpx, lrow, g);
}

// Repack [Co][Ci][K][K] (fp32 or bf16) to bf16 [Co_pad][K*K][Ci_pad], zeros
// in the padding.
template <typename TW>
__global__ void conv2d_pack_kernel(const TW* __restrict__ w, int Co, int Ci, int KK, int Co_pad, int Ci_pad,
                                   uint16_t* __restrict__ out) {
    const int64_t total = (int64_t)Co_pad * KK * Ci_pad;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int ci = (int)(i % Ci_pad);
        const int64_t r = i / Ci_pad;
        const int tap = (int)(r % KK), co = (int)(r / KK);
        float v = 0.f;
        if (co < Co && ci < Ci) v = load_in<TW>(w + ((int64_t)co * Ci + ci) * KK + tap);
        out[i] = (uint16_t)(pack_bf16x2(v, 0.f) & 0xFFFFu);
    }
}

int64_t pad_to(int64_t v, int64_t m) { return (v + m - 1) / m * m; }

}  // namespace
}  // namespace dit

extern "C" size_t dt_conv2d_packed_bytes(int64_t Co, int64_t Ci, int64_t K) {
    if (Co <= 0 || Ci <= 0 || (K != 1 && K != 3)) return 0;
    return (size_t)(dit::pad_to(Co, dit::kTileCo) * K * K * dit::pad_to(Ci, dit::kCi) * 2);
}

extern "C" int dt_conv2d_pack_weights(const void* w, int32_t w_type, int64_t Co, int64_t Ci, int64_t K,
                                      void* packed, dt_stream_t stream) {
    using namespace dit;
    DT_REQUIRE(Co > 0 && Ci > 0 && (K == 1 || K == 3), "dt_conv2d_pack_weights: Co, Ci > 0 and K in {1, 3}");
    DT_REQUIRE(w_type == DT_TYPE_F32 || w_type == DT_TYPE_BF16, "dt_conv2d_pack_weights: w_type %d unsupported",
               w_type);
    DT_REQUIRE(w && packed, "dt_conv2d_pack_weights: null pointer");
    DT_REQUIRE(Co < (1 << 24) && Ci < (1 << 24), "dt_conv2d_pack_weights: too many channels");
    const int co_pad = (int)pad_to(Co, kTileCo), ci_pad = (int)pad_to(Ci, kCi), kk = (int)(K * K);
    const int64_t total = (int64_t)co_pad * kk * ci_pad;
    const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 4096);
    if (w_type == DT_TYPE_F32)
        hipLaunchKernelGGL((conv2d_pack_kernel<float>), dim3(grid), dim3(256), 0, (hipStream_t)stream,
                           (const float*)w, (int)Co, (int)Ci, kk, co_pad, ci_pad, (uint16_t*)packed);
    else
        hipLaunchKernelGGL((conv2d_pack_kernel<bf16>), dim3(grid), dim3(256), 0, (hipStream_t)stream,
                           (const bf16*)w, (int)Co, (int)Ci, kk, co_pad, ci_pad, (uint16_t*)packed);
    return check_launch("dt_conv2d_pack_weights");
}

namespace dit {
namespace {

// Tile geometry of an output image of Hs x Ws: TC = 128, 64, 32 or 16 columns.
void conv_geometry(int64_t Hs, int64_t Ws, int* TR, int* TC, int64_t* tiles_w, int64_t* tiles_h) {
    *TC = Ws >= 128 ? 128 : Ws >= 64 ? 64 : Ws >= 32 ? 32 : 16;
    *TR = kTilePx / *TC;
    *tiles_w = (Ws + *TC - 1) / *TC;
    *tiles_h = (Hs + *TR - 1) / *TR;
}

int conv_launch(const void* x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void* packed_w, int64_t Co,
                int64_t K, int32_t upscale2, const float* bias, void* y, int32_t io_type, float4* stats,
                int64_t groups, hipStream_t st, const char* what) {
    DT_REQUIRE(is_io_type(io_type), "%s: io_type %d unsupported", what, io_type);
    DT_REQUIRE(N > 0 && Ci > 0 && H > 0 && W > 0 && Co > 0, "%s: bad shape", what);
    DT_REQUIRE(K == 1 || K == 3, "%s: kernel size %lld unsupported (1 or 3)", what, (long long)K);
    DT_REQUIRE(x && packed_w && y, "%s: null pointer", what);
    DT_REQUIRE(aligned16(packed_w), "%s: packed weights must be 16-byte aligned", what);
    const int64_t Hs = upscale2 ? 2 * H : H, Ws = upscale2 ? 2 * W : W;
    DT_REQUIRE(N < 65536 && Co < (1 << 24) && Ci < (1 << 24) && Hs * Ws < (1ll << 31) &&
                   N * Ci * H * W < (1ll << 40),
               "%s: shape too large", what);
    ConvArgs a{};
    a.x = x;
    a.w = (const uint16_t*)packed_w;
    a.bias = bias;
    a.y = y;
    a.N = (int)N; a.Ci = (int)Ci; a.H = (int)H; a.W = (int)W;
    a.Co = (int)Co; a.K = (int)K; a.up2 = upscale2 ? 1 : 0;
    a.Hs = (int)Hs; a.Ws = (int)Ws;
    a.Ci_pad = (int)pad_to(Ci, kCi);
    a.KK = (int)(K * K);
    int64_t tiles_w, tiles_h;
    conv_geometry(Hs, Ws, &a.TR, &a.TC, &tiles_w, &tiles_h);
    a.tiles_w = (int)tiles_w;
    a.stats = stats;
    a.G = (int)groups;
    a.cg = groups > 0 ? (int)(Co / groups) : 0;
    DT_REQUIRE(tiles_h * tiles_w < (1ll << 31), "%s: too many tiles", what);
    const dim3 grid((unsigned)(tiles_h * tiles_w), (unsigned)((Co + kTileCo - 1) / kTileCo), (unsigned)N);
#define DT_CONV_LAUNCH(TT, KS, ST) hipLaunchKernelGGL((conv2d_kernel<TT, KS, ST>), grid, dim3(256), 0, st, a)
    if (io_type == DT_TYPE_F32) {
        if (K == 3) { if (stats) DT_CONV_LAUNCH(float, 3, true); else DT_CONV_LAUNCH(float, 3, false); }
        else { if (stats) DT_CONV_LAUNCH(float, 1, true); else DT_CONV_LAUNCH(float, 1, false); }
    } else {
        if (K == 3) { if (stats) DT_CONV_LAUNCH(bf16, 3, true); else DT_CONV_LAUNCH(bf16, 3, false); }
        else { if (stats) DT_CONV_LAUNCH(bf16, 1, true); else DT_CONV_LAUNCH(bf16, 1, false); }
    }
#undef DT_CONV_LAUNCH
    return check_launch(what);
}

}  // namespace
}  // namespace dit

extern "C" int dt_conv2d(const void* x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void* packed_w,
                         int64_t Co, int64_t K, int32_t upscale2, const float* bias, void* y, int32_t io_type,
                         dt_stream_t stream) {
    return dit::conv_launch(x, N, Ci, H, W, packed_w, Co, K, upscale2, bias, y, io_type, nullptr, 0,
                            (hipStream_t)stream, "dt_conv2d");
}

extern "C" size_t dt_conv2d_gn_stats_bytes(int64_t N, int64_t Co, int64_t OH, int64_t OW, int64_t groups) {
    if (N <= 0 || Co <= 0 || OH <= 0 || OW <= 0 || groups <= 0 || Co % groups) return 0;
    int tr, tc;
    int64_t tw, th;
    dit::conv_geometry(OH, OW, &tr, &tc, &tw, &th);
    return (size_t)(dit::gn_tile_stats_head_bytes(N, groups) + N * groups * th * tw * 16);
}

extern "C" int dt_conv2d_gn(const void* x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void* packed_w,
                            int64_t Co, int64_t K, int32_t upscale2, const float* bias, void* y, int64_t groups,
                            void* stats, size_t stats_bytes, int32_t io_type, dt_stream_t stream) {
    using namespace dit;
    DT_REQUIRE(groups > 0 && Co % groups == 0, "dt_conv2d_gn: Co %lld not a multiple of groups %lld",
               (long long)Co, (long long)groups);
    const int64_t cg = Co / groups;
    DT_REQUIRE(cg <= kTileCo && kTileCo % cg == 0,
               "dt_conv2d_gn: %lld channels per group must divide %d", (long long)cg, kTileCo);
    DT_REQUIRE(stats && ((uintptr_t)stats & 15) == 0, "dt_conv2d_gn: stats must be 16-byte aligned");
    const int64_t Hs = upscale2 ? 2 * H : H, Ws = upscale2 ? 2 * W : W;
    const size_t need = dt_conv2d_gn_stats_bytes(N, Co, Hs, Ws, groups);
    DT_REQUIRE(need > 0 && stats_bytes >= need, "dt_conv2d_gn: stats buffer too small (%zu < %zu)", stats_bytes,
               need);
    DT_REQUIRE(N * groups < 65536, "dt_conv2d_gn: N*groups must be < 65536");
    hipStream_t st = (hipStream_t)stream;
    float4* recs = (float4*)((char*)stats + gn_tile_stats_head_bytes(N, groups));
    int rc = conv_launch(x, N, Ci, H, W, packed_w, Co, K, upscale2, bias, y, io_type, recs, groups, st,
                         "dt_conv2d_gn");
    if (rc) return rc;
    int tr, tc;
    int64_t tw, th;
    conv_geometry(Hs, Ws, &tr, &tc, &tw, &th);
    return gn_tile_stats_finalize(stats, N, groups, th * tw, st);
}
