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
#include "capi_util.hpp"
#include "common.hpp"

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
};

template <typename TI>
__device__ __forceinline__ float load_in(const TI* p);
template <>
__device__ __forceinline__ float load_in<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_in<bf16>(const bf16* p) {
    return __uint_as_float((uint32_t)*reinterpret_cast<const uint16_t*>(p) << 16);
}

template <typename T, int K>
__global__ __launch_bounds__(256) void conv2d_kernel(const ConvArgs a) {
    constexpr int KK = K * K, PAD = (K - 1) / 2;
    constexpr int W_BYTES = kTileCo * KK * kRec;
    // input patch: up to (TR + K - 1) x (TC + K - 1) pixels; TR x TC = 128
    constexpr int X_MAX = (128 + K - 1) * (1 + K - 1) > (16 + K - 1) * (8 + K - 1)
                              ? (128 + K - 1) * (1 + K - 1) : (16 + K - 1) * (8 + K - 1);
    __shared__ __attribute__((aligned(16))) uint8_t smem[W_BYTES + X_MAX * kRec];
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

extern "C" int dt_conv2d(const void* x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void* packed_w,
                         int64_t Co, int64_t K, int32_t upscale2, const float* bias, void* y, int32_t io_type,
                         dt_stream_t stream) {
    using namespace dit;
    DT_REQUIRE(is_io_type(io_type), "dt_conv2d: io_type %d unsupported", io_type);
    DT_REQUIRE(N > 0 && Ci > 0 && H > 0 && W > 0 && Co > 0, "dt_conv2d: bad shape");
    DT_REQUIRE(K == 1 || K == 3, "dt_conv2d: kernel size %lld unsupported (1 or 3)", (long long)K);
    DT_REQUIRE(x && packed_w && y, "dt_conv2d: null pointer");
    DT_REQUIRE(aligned16(packed_w), "dt_conv2d: packed weights must be 16-byte aligned");
    const int64_t Hs = upscale2 ? 2 * H : H, Ws = upscale2 ? 2 * W : W;
    DT_REQUIRE(N < 65536 && Co < (1 << 24) && Ci < (1 << 24) && Hs * Ws < (1ll << 31) &&
                   N * Ci * H * W < (1ll << 40),
               "dt_conv2d: shape too large");
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
    a.TC = Ws >= 128 ? 128 : Ws >= 64 ? 64 : Ws >= 32 ? 32 : 16;
    a.TR = kTilePx / a.TC;
    a.tiles_w = (int)((Ws + a.TC - 1) / a.TC);
    const int64_t tiles_h = (Hs + a.TR - 1) / a.TR;
    DT_REQUIRE(tiles_h * a.tiles_w < (1ll << 31), "dt_conv2d: too many tiles");
    const dim3 grid((unsigned)(tiles_h * a.tiles_w), (unsigned)((Co + kTileCo - 1) / kTileCo), (unsigned)N);
    hipStream_t st = (hipStream_t)stream;
    if (io_type == DT_TYPE_F32) {
        if (K == 3) hipLaunchKernelGGL((conv2d_kernel<float, 3>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((conv2d_kernel<float, 1>), grid, dim3(256), 0, st, a);
    } else {
        if (K == 3) hipLaunchKernelGGL((conv2d_kernel<bf16, 3>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((conv2d_kernel<bf16, 1>), grid, dim3(256), 0, st, a);
    }
    return check_launch("dt_conv2d");
}
