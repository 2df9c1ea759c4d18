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
    // Residual epilogue (ConvFold): 1: y = res + conv; 2: y = (res +
    // conv) * res_scale.  res is an NCHW tensor of the output's shape and type.
    const void* res;
    int res_mode;
    float res_scale;
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

// The residual epilogue of ResnetBlock2D's `(input + hidden) /
// output_scale_factor` for output pixel (oh, ow): its accumulator rows
// acc[j][i][r] (j = 0, 1) are output channels co_base + 32 j + 8 (r / 4) +
// (r % 4) of sample n.  Each value is conv + bias, then + the residual, then
// (res_mode 2) * res_scale, rounded to T where the graph stores the node
// (the conv output, the ADD; the SCALE by the store itself), so the fused
// epilogue equals the nodes.  Each j's 16 residual values are loaded before
// its first store: the output may sit on its own residual, but each element
// is read and then written by this lane alone, so the loads need not wait
// on earlier stores (two memory round trips per pixel instead of one per
// element).
template <typename T, int FN>
__device__ __forceinline__ void conv_store_residual(const ConvArgs& a, T* y, const f32x16_t (&acc)[2][FN], int i,
                                                    int co_base, int oh, int ow, int n) {
    const T* res = reinterpret_cast<const T*>(a.res) + (int64_t)n * a.Co * a.Hs * a.Ws;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        float rv[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int co = co_base + 32 * j + 8 * (r >> 2) + (r & 3);
            rv[r] = co < a.Co ? Io<T>::get(res + ((int64_t)co * a.Hs + oh) * a.Ws + ow) : 0.f;
        }
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int co = co_base + 32 * j + 8 * (r >> 2) + (r & 3);
            if (co >= a.Co) continue;
            float v = acc[j][i][r];
            if (a.bias) v = add_rn(v, a.bias[co]);
            v = add_rn(rv[r], stored_value<T>(v));
            if (a.res_mode == 2) v = mul_rn(stored_value<T>(v), a.res_scale);
            Io<T>::put(y + ((int64_t)co * a.Hs + oh) * a.Ws + ow, v);
        }
    }
}

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
        const bool valid = (p >> __builtin_ctz(a.TC)) < rows_valid && (p & (a.TC - 1)) < cols_valid;
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
    const bool full = vp == kTilePx;
    const int lt = __builtin_ctz(a.TC);  // TC is a power of two
    // Sum over the tpg threads of a group: xor shuffles when the group lies in
    // one wave (tpg <= 64, every decoder shape), else through LDS.
    auto seg_sum = [&](float v) {
        if (tpg <= kWave) {
            for (int o = tpg / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
            return v;
        }
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
    if (full) {
        for (int e = ti; e < n_el; e += tpg) {
            const float d = gv[e] - mean;
            s2 += d * d;
        }
    } else {
        for (int e = ti; e < n_el; e += tpg) {
            const int p = e & (kTilePx - 1);
            if ((p >> lt) < rows_valid && (p & (a.TC - 1)) < cols_valid) {
                const float d = gv[e] - mean;
                s2 += d * d;
            }
        }
    }
    const float m2 = seg_sum(s2);
    const int grp = co0 / a.cg + gi;
    if (ti == 0 && grp < a.G)
        a.stats[((int64_t)blockIdx.z * a.G + grp) * gridDim.x + blockIdx.x] =
            make_float4(mean, m2, (float)(a.cg * vp), 0.f);
}

// The same statistics straight from the accumulators, for CG = 4 .. 64
// channels per group (the decoder's 4, 8 and 16): each lane sums the rows of
// its FN pixels that share a group ("slots": the lane's 32 rows are
// 32 j + 8 q + 4 g + t of its wave's 64), xor-shuffles the slot sums across
// the 32 (CG = 4) or 64 lanes holding the group, and the two waves covering
// the tile's two pixel halves (wave and wave ^ 1) add theirs through LDS; then the same for
// M2 around the group mean.  Two barriers, no LDS tile.
template <typename T, int CG, int FN = 2>
__device__ __forceinline__ void conv_group_stats_reg(const ConvArgs& a, const f32x16_t (&acc)[2][FN], float* red,
                                                     int co0, int oh0, int ow0, int wco, int wpx, int lrow, int g,
                                                     int wave) {
    constexpr int S = CG <= 8 ? 8 : CG == 16 ? 4 : CG == 32 ? 2 : 1;  // slots per lane
    constexpr int WIDTH = CG == 4 ? 32 : 64;                            // lanes holding one slot's group
    const int rows_valid = min(a.TR, a.Hs - oh0), cols_valid = min(a.TC, a.Ws - ow0);
    const int lt = __builtin_ctz(a.TC);
    bool valid[FN];
#pragma unroll
    for (int i = 0; i < FN; ++i) {
        const int p = wpx + 32 * i + lrow;
        valid[i] = (p >> lt) < rows_valid && (p & (a.TC - 1)) < cols_valid;
    }
    // The stored values (bias added, rounded to T).
    float v[2][FN][16];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
            const int co = co0 + wco + 32 * j + 8 * (r >> 2) + 4 * g + (r & 3);
            const float bv = a.bias && co < a.Co ? a.bias[co] : 0.f;
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                float t = acc[j][i][r];
                if (a.bias) t = add_rn(t, bv);
                v[j][i][r] = stored_value<T>(t);
            }
        }
    auto slot_of = [](int j, int q) { return CG <= 8 ? 4 * j + q : CG == 16 ? 2 * j + (q >> 1) : CG == 32 ? j : 0; };
    auto entry = [&](int s) { return CG == 4 ? 2 * s + g : s; };  // LDS entry of slot s
    const int vp = rows_valid * cols_valid;
    // Pass 1: sums.
    float part[S];
#pragma unroll
    for (int s = 0; s < S; ++s) part[s] = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
            for (int i = 0; i < FN; ++i)
                if (valid[i]) part[slot_of(j, r >> 2)] += v[j][i][r];
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int o = WIDTH / 2; o > 0; o >>= 1) part[s] += __shfl_xor(part[s], o, kWave);
    if (lrow == 0 && (CG == 4 || g == 0))
#pragma unroll
        for (int s = 0; s < S; ++s) red[wave * 16 + entry(s)] = part[s];
    __syncthreads();
    float mean[S];
#pragma unroll
    for (int s = 0; s < S; ++s)
        mean[s] = (red[wave * 16 + entry(s)] + red[(wave ^ 1) * 16 + entry(s)]) / (float)(CG * vp);
    __syncthreads();
    // Pass 2: M2 around the group mean.
#pragma unroll
    for (int s = 0; s < S; ++s) part[s] = 0.f;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r)
#pragma unroll
            for (int i = 0; i < FN; ++i)
                if (valid[i]) {
                    const float d = v[j][i][r] - mean[slot_of(j, r >> 2)];
                    part[slot_of(j, r >> 2)] += d * d;
                }
#pragma unroll
    for (int s = 0; s < S; ++s)
#pragma unroll
        for (int o = WIDTH / 2; o > 0; o >>= 1) part[s] += __shfl_xor(part[s], o, kWave);
    if (lrow == 0 && (CG == 4 || g == 0))
#pragma unroll
        for (int s = 0; s < S; ++s) red[wave * 16 + entry(s)] = part[s];
    __syncthreads();
    if ((wave & 1) == 0 && lrow == 0 && (CG == 4 || g == 0)) {
#pragma unroll
        for (int s = 0; s < S; ++s) {
            const float m2 = red[wave * 16 + entry(s)] + red[(wave ^ 1) * 16 + entry(s)];
            // the slot's group: its first row wco + (32 j + 8 q + 4 g) / CG * CG
            const int grp = co0 / CG + wco / CG + (CG == 4 ? 2 * s + g : s);
            if (grp < a.G)
                a.stats[((int64_t)blockIdx.z * a.G + grp) * gridDim.x + blockIdx.x] =
                    make_float4(mean[s], m2, (float)(CG * vp), 0.f);
        }
    }
}

template <typename T, int K, bool STATS, bool RES>
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
        if constexpr (RES) {
            conv_store_residual<T, 2>(a, y, acc, i, co0 + wco + 4 * g, oh, ow, n);
            continue;
        }
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
    if constexpr (STATS) {
        float* red = reinterpret_cast<float*>(smem);  // free after the main loop's last barrier
        switch (a.cg) {
            case 4: conv_group_stats_reg<T, 4>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
            case 8: conv_group_stats_reg<T, 8>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
            case 16: conv_group_stats_reg<T, 16>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
            case 32: conv_group_stats_reg<T, 32>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
            case 64: conv_group_stats_reg<T, 64>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
            default: conv_group_stats<T>(a, acc, smem, co0, oh0, ow0, wco, wpx, lrow, g); break;
        }
    }
}

// ---- with a workspace (3x3; 1x1 on bf16): channel-last input, direct
// global -> LDS DMA.  Measured on gfx950 (bf16, 3x3, Co = Ci, channel-last
// copy included): [1,512,128,128] 693, [1,512,256,256] 846, [1,256,512,512]
// 674, [1,128,1024,1024] 497 TFLOP/s; the register-staged kernel 99-125.
// The input is first transposed to bf16 NHWC with channels zero-padded to a
// multiple of 16 (to_nhwc16_kernel, one bandwidth-bound pass, which can also
// apply a GroupNorm + SiLU), so a 16-channel slice of one pixel is a
// contiguous 32-byte record and both operands stream into LDS by
// global_load_lds with no per-element work: the input patch of a 256- or
// 512-pixel tile (every lane computes its own source pixel, which also
// applies the nearest 2x upscale and sends out-of-image taps to a zeroed
// 256-byte tail of the workspace) and the [128 co][K*K] weight records.  Two
// LDS stages of 16 channels, filled one chunk ahead; four waves of 64 co x
// 32 FN px (2 x FN MFMA 32x32x16 per tap).  The DMA source swaps each
// 32-byte record's two 16-byte units by the rule below (kSwzBit), so
// consecutive records read distinct banks.  The output leaves through LDS
// (conv_store_lds).
constexpr int kCi2 = 16, kRec2 = 32;
// A record's two 16-byte units are swapped when bit 3 of its pixel (or
// output-channel) index is set.  Record r's unit u then starts at bank
// 8 (r mod 8) + 4 (u ^ bit3(r)) of 64, so any 16 consecutive records -- the
// 16 lanes one ds_read_b128 cycle serves -- cover all 64 banks.  (Swapping
// on bit 2 repeated banks every 8 records: SQ_LDS_BANK_CONFLICT was half of
// SQ_LDS_IDX_ACTIVE.)
constexpr int kSwzBit = 3;
// DMA lanes per X stage: 2 per record, up to the 10 x 34 records of an
// 8 x 32 tile (the 16 x 16 tile needs 18 x 18).  Lanes past the patch read
// the zero tail, so the count is kept to the largest patch.
constexpr int kXLanesMax3 = 3 * 256;
static_assert(2 * (8 + 2) * (32 + 2) <= kXLanesMax3 && 2 * (16 + 2) * (16 + 2) <= kXLanesMax3,
              "X DMA lanes must cover the 3x3 patch of every tile shape conv_geometry2 picks");
// The same for the 512-pixel tiles (16 x 32, or 32 x 16 on narrow images).
constexpr int kXLanesMax3x2 = 5 * 256;
static_assert(2 * (16 + 2) * (32 + 2) <= kXLanesMax3x2 && 2 * (32 + 2) * (16 + 2) <= kXLanesMax3x2,
              "X DMA lanes must cover the 3x3 patch of every 512-pixel tile");

// GroupNorm applied by the channel-last copy: (mean, rstd) per (n, group),
// the per-channel affine (or null), cg channels per group, the SiLU flag.
struct CopyGn {
    const float2* mr;
    const float* w;
    const float* b;
    int G, cg, silu;
};

// NCHW (fp32 or bf16) -> bf16 NHWC with C16 channels (zeros past C), over
// the flattened H*W plane in tiles of 64 pixels x 64 channels: 16-byte loads
// along the pixels of each channel (VEC; scalar when the plane is not a
// multiple of 8 pixels), a transpose through LDS, and 16-byte stores of 8
// channels of one pixel.  Block (0, 0, 0) also zeroes the 256-byte tail the
// conv reads for out-of-image taps.  GN: each loaded value first becomes
// silu((x - mean) * (rstd * w_c) + b_c), the very expression (and rounding)
// of the GroupNorm apply pass, so the copy holds what copying that pass's
// output would give.
template <typename TI, bool VEC, bool GN>
__global__ __launch_bounds__(256) void to_nhwc16_kernel(const TI* __restrict__ x, int C, int64_t HW, int C16,
                                                        uint16_t* __restrict__ out, int64_t tail_offset,
                                                        CopyGn gn) {
    __shared__ uint16_t t[64][64 + 2];  // [channel][pixel] (+2: spread the per-pixel column reads)
    const int64_t p0 = (int64_t)blockIdx.x * 64;
    const int c0 = blockIdx.y * 64, n = blockIdx.z;
    const TI* xn = x + (int64_t)n * C * HW;
    uint16_t* on = out + (int64_t)n * HW * C16;
    constexpr int EPV = VEC ? 16 / (int)sizeof(TI) : 1;  // pixels per load
    constexpr int VPR = 64 / EPV;                          // loads per channel row
    for (int u = threadIdx.x; u < 64 * VPR; u += 256) {
        const int c = u / VPR, q = u - c * VPR;
        const int64_t p = p0 + q * EPV;
        float v[EPV];
        if (c0 + c < C && p < HW) {
            if constexpr (VEC) {
                Io<TI>::load(xn + (int64_t)(c0 + c) * HW + p, v);
            } else {
                v[0] = load_in<TI>(xn + (int64_t)(c0 + c) * HW + p);
            }
            if constexpr (GN) {
                const int ch = c0 + c;
                const float2 mr = gn.mr[n * gn.G + ch / gn.cg];
                const float sa = gn.w ? mr.y * gn.w[ch] : mr.y, bc = gn.b ? gn.b[ch] : 0.0f;
#pragma unroll
                for (int k = 0; k < EPV; ++k) {
                    const float t = __builtin_fmaf(v[k] - mr.x, sa, bc);
                    v[k] = gn.silu ? silu_fast(t) : t;
                }
            }
        } else {
#pragma unroll
            for (int k = 0; k < EPV; ++k) v[k] = 0.f;
        }
#pragma unroll
        for (int k = 0; k < EPV; ++k) t[c][q * EPV + k] = (uint16_t)(pack_bf16x2(v[k], 0.f) & 0xFFFFu);
    }
    __syncthreads();
    for (int u = threadIdx.x; u < 64 * 8; u += 256) {
        const int px = u >> 3, part = u & 7;  // pixel, 8-channel unit
        const int64_t p = p0 + px;
        const int c = c0 + part * 8;
        if (p >= HW || c >= C16) continue;
        uint32_t w[4];
#pragma unroll
        for (int k = 0; k < 4; ++k)
            w[k] = (uint32_t)t[part * 8 + 2 * k][px] | ((uint32_t)t[part * 8 + 2 * k + 1][px] << 16);
        *reinterpret_cast<uint4*>(on + p * C16 + c) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    if (blockIdx.x == 0 && blockIdx.y == 0 && blockIdx.z == 0 && threadIdx.x < 16)
        reinterpret_cast<uint4*>(out + tail_offset)[threadIdx.x] = make_uint4(0, 0, 0, 0);
}

struct Conv2Extra {
    const uint16_t* xh;  // NHWC bf16 [N][H][W][C16]
    const uint16_t* zero;  // 256 zero bytes
    int C16, Cp32;       // channels of xh; Ci_pad of the packed weights
    int lt;              // log2(TC)
};

__device__ __forceinline__ void dma16(const void* src, void* lds) { __builtin_amdgcn_global_load_lds(src, lds, 16, 0, 0); }

template <int N_OUT>
__device__ __forceinline__ void conv_wait_vm() {
    // s_waitcnt vmcnt(N_OUT) with expcnt / lgkmcnt left at their maxima.
    __builtin_amdgcn_s_waitcnt((N_OUT & 15) | ((N_OUT >> 4) << 14) | 0x0F70);
}

// The epilogue of the DMA kernel's 128-channel x 256-pixel tile, through
// LDS, in two passes over the accumulator halves j (64 output channels
// each).  Each lane parks its conv + bias values, rounded to T as the graph
// stores the conv node, in LDS as [64 channels][256 pixels]; the block then
// writes the pass in 16-byte pieces along the image rows (the lanes' own
// values would be 2-byte stores).  RES adds the residual epilogue of
// ResnetBlock2D's `(input + hidden) / output_scale_factor`: per piece the
// residual (loaded before the LDS stage, so its latency overlaps it), the
// ADD rounded to T, the SCALE (res_mode 2), one store.  A piece is read and
// written by one thread only, so the output may sit on the residual.
// The epilogue's LDS: 64 output-channel rows of the tile's 64 FN pixels,
// padded by 8 elements; the DMA kernel's shared array is at least this large.
template <int FN>
constexpr int epi_stride() { return 64 * FN + 8; }
template <typename T, int FN>
constexpr int epi_lds_bytes() { return 64 * epi_stride<FN>() * (int)sizeof(T); }

template <typename T, bool RES, int FN>
__device__ __forceinline__ void conv_store_lds(const ConvArgs& a, const f32x16_t (&acc)[2][FN], uint8_t* smem,
                                               int co0, int oh0, int ow0, int wco, int wpx, int lrow, int g, int lt,
                                               int n) {
    constexpr int E = Io<T>::EPV;             // elements per 16-byte piece
    constexpr int S = epi_stride<FN>();       // LDS row stride in elements (bank-spread rows)
    constexpr int RP = 64 * FN / E;           // pieces per pixel row
    constexpr int PIECES = 64 * RP / 256;     // pieces per thread and pass
    T* lds = reinterpret_cast<T*>(smem);
    const int tid = threadIdx.x, tcm = (1 << lt) - 1;
    const int64_t plane = (int64_t)a.Hs * a.Ws;
    const T* res = RES ? reinterpret_cast<const T*>(a.res) + (int64_t)n * a.Co * plane : nullptr;
    T* y = reinterpret_cast<T*>(a.y) + (int64_t)n * a.Co * plane;
    const bool vec = a.Ws % E == 0 && (!RES || (reinterpret_cast<uintptr_t>(a.res) & 15) == 0) &&
                     (reinterpret_cast<uintptr_t>(a.y) & 15) == 0;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        uint4 rv[PIECES];
#pragma unroll
        for (int k = 0; k < PIECES && RES; ++k) {
            const int c = tid + 256 * k, pr = c / RP, px = (c % RP) * E;
            const int co = co0 + (pr >> 5) * 64 + 32 * j + (pr & 31);
            const int oh = oh0 + (px >> lt), ow = ow0 + (px & tcm);
            rv[k] = make_uint4(0, 0, 0, 0);
            if (co >= a.Co || oh >= a.Hs || ow >= a.Ws) continue;
            const T* src = res + co * plane + (int64_t)oh * a.Ws + ow;
            if (vec) {
                rv[k] = ld_stream(src);
            } else {
                float t[E];
#pragma unroll
                for (int q = 0; q < E; ++q) t[q] = ow + q < a.Ws ? Io<T>::get(src + q) : 0.f;
                rv[k] = Io<T>::pack(t);
            }
        }
#pragma unroll
        for (int i = 0; i < FN; ++i) {
            float v[16];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int q = 8 * (r >> 2) + 4 * g + (r & 3), co = co0 + wco + 32 * j + q;
                v[r] = acc[j][i][r];
                if (a.bias && co < a.Co) v[r] = add_rn(v[r], a.bias[co]);
            }
            if constexpr (sizeof(T) == 2) {
                // Lanes 2k and 2k + 1 hold pixels p and p + 1.  For each
                // pair of adjacent channels (r, r + 1) they swap one value
                // (DPP lane ^ 1), so the even lane writes channel r's and
                // the odd lane channel r + 1's two pixels as one dword.
                const bool odd = lrow & 1;
                const int p = wpx + 32 * i + (lrow & ~1);
#pragma unroll
                for (int r = 0; r < 16; r += 2) {
                    const float mine = odd ? v[r + 1] : v[r];
                    const float other = dpp_f32<0xB1>(odd ? v[r] : v[r + 1]);
                    const int q = 8 * (r >> 2) + 4 * g + (r & 3) + (odd ? 1 : 0);
                    *reinterpret_cast<uint32_t*>(lds + ((wco >> 6) * 32 + q) * S + p) =
                        odd ? pack_bf16x2(other, mine) : pack_bf16x2(mine, other);
                }
            } else {
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    const int q = 8 * (r >> 2) + 4 * g + (r & 3);
                    Io<T>::put(lds + ((wco >> 6) * 32 + q) * S + wpx + 32 * i + lrow, v[r]);
                }
            }
        }
        __syncthreads();
#pragma unroll
        for (int k = 0; k < PIECES; ++k) {
            const int c = tid + 256 * k, pr = c / RP, px = (c % RP) * E;
            const int co = co0 + (pr >> 5) * 64 + 32 * j + (pr & 31);
            const int oh = oh0 + (px >> lt), ow = ow0 + (px & tcm);
            if (co >= a.Co || oh >= a.Hs || ow >= a.Ws) continue;
            T* dst = y + co * plane + (int64_t)oh * a.Ws + ow;
            const uint4 hv = *reinterpret_cast<const uint4*>(lds + pr * S + px);
            if constexpr (!RES) {
                if (vec) {
                    st_stream(dst, hv);
                } else {
#pragma unroll
                    for (int q = 0; q < E; ++q)
                        if (ow + q < a.Ws) dst[q] = lds[pr * S + px + q];
                }
                continue;
            }
            float h[E], r[E];
            Io<T>::unpack(hv, h);
            Io<T>::unpack(rv[k], r);
#pragma unroll
            for (int q = 0; q < E; ++q) h[q] = add_rn(r[q], h[q]);
            if (a.res_mode == 2) {
                Io<T>::round(h);
#pragma unroll
                for (int q = 0; q < E; ++q) h[q] = mul_rn(h[q], a.res_scale);
            }
            if (vec) {
                st_stream(dst, Io<T>::pack(h));
            } else {
#pragma unroll
                for (int q = 0; q < E; ++q)
                    if (ow + q < a.Ws) Io<T>::put(dst + q, h[q]);
            }
        }
        __syncthreads();  // the next pass reuses the LDS rows
    }
}

// FN: 32-pixel MFMA columns per wave, 4 (a 256-pixel tile of 8 x 32) or 8
// (512 pixels, 16 x 32, halving the weight DMA per output pixel, for convs
// with enough tiles to fill the chip).
template <typename T, int K, bool STATS, bool RES, int FN>
__global__ __launch_bounds__(256) void conv2d_dma_kernel(const ConvArgs a, const Conv2Extra e) {
    static_assert(K == 3 || K == 1, "the DMA kernel takes 3x3 and 1x1 patches");
    static_assert(FN == 4 || (FN == 8 && !STATS && !RES), "512-pixel tiles carry no statistics or residual epilogue");
    constexpr int KK = K * K, PAD = (K - 1) / 2;
    constexpr int XL = FN == 4 ? kXLanesMax3 : kXLanesMax3x2;  // X DMA lanes per stage
    constexpr int NX = XL / 256, NW = 2 * kTileCo * KK / 256;  // DMA instructions per wave per stage
    constexpr int XB = XL * 16, WB = kTileCo * KK * kRec2, STAGE = XB + WB;
    constexpr int QD = NX + NW;
    // the two DMA stages, then the epilogue's rows (larger for 1x1 patches)
    constexpr int SMEM = 2 * STAGE > epi_lds_bytes<T, FN>() ? 2 * STAGE : epi_lds_bytes<T, FN>();
    __shared__ __attribute__((aligned(16))) uint8_t smem[SMEM];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int n = blockIdx.z, co0 = blockIdx.y * kTileCo;
    const int th = blockIdx.x / a.tiles_w, tw = blockIdx.x - th * a.tiles_w;
    const int oh0 = th * a.TR, ow0 = tw * a.TC;
    const int PC = a.TC + K - 1, npatch = (a.TR + K - 1) * PC;
    const int wco = (wave >> 1) * 64, wpx = (wave & 1) * 32 * FN;
    const int lrow = lane & 31, g = lane >> 5;

    // DMA sources, fixed for the whole K loop up to the channel offset.
    const uint16_t* xsrc[NX];
    int xstep[NX];  // 1 for an in-image record (advances with the channel chunk), 0 for the zero tail
#pragma unroll
    for (int m = 0; m < NX; ++m) {
        const int L = (m * 4 + wave) * 64 + lane, rec = L >> 1, u = L & 1;
        const uint16_t* src = e.zero;
        xstep[m] = 0;
        if (rec < npatch) {
            const int pr = rec / PC, pc = rec - pr * PC;
            const int ih = oh0 + pr - PAD, iw = ow0 + pc - PAD;
            if (ih >= 0 && ih < a.Hs && iw >= 0 && iw < a.Ws) {
                const int sh = a.up2 ? ih >> 1 : ih, sw = a.up2 ? iw >> 1 : iw;
                const int su = u ^ ((rec >> kSwzBit) & 1);
                src = e.xh + (((int64_t)n * a.H + sh) * a.W + sw) * e.C16 + su * 8;
                xstep[m] = 1;
            }
        }
        xsrc[m] = src;
    }
    const uint16_t* wsrc[NW];
#pragma unroll
    for (int m = 0; m < NW; ++m) {
        const int L = (m * 4 + wave) * 64 + lane, rec = L >> 1, u = L & 1;
        const int co = rec / KK, tap = rec - co * KK;
        const int su = u ^ ((co >> kSwzBit) & 1);
        wsrc[m] = a.w + ((int64_t)(co0 + co) * KK + tap) * e.Cp32 + su * 8;
    }
    auto issue = [&](int c0, int s) {
        uint8_t* st = smem + s * STAGE;
#pragma unroll
        for (int m = 0; m < NX; ++m)  // out-of-image taps read the zero tail at every chunk
            dma16(xsrc[m] + xstep[m] * c0, st + (m * 4 + wave) * 64 * 16);
#pragma unroll
        for (int m = 0; m < NW; ++m) dma16(wsrc[m] + c0, st + XB + (m * 4 + wave) * 64 * 16);
    };

    f32x16_t acc[2][FN];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int i = 0; i < FN; ++i)
#pragma unroll
            for (int q = 0; q < 16; ++q) acc[j][i][q] = 0.f;

    int pbase[FN];
#pragma unroll
    for (int i = 0; i < FN; ++i) {
        const int p = wpx + 32 * i + lrow;
        pbase[i] = (p >> e.lt) * PC + (p & (a.TC - 1));
    }
    int wrec[2], wsw[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int co = wco + 32 * j + lrow;
        wrec[j] = co * KK;
        wsw[j] = (g ^ ((co >> kSwzBit) & 1)) << 4;
    }

    const int nch = e.C16 / kCi2;
    issue(0, 0);
    if (nch > 1) issue(kCi2, 1);
    for (int ch = 0; ch < nch; ++ch) {
        if (ch + 1 < nch) conv_wait_vm<QD>();
        else conv_wait_vm<0>();
        __builtin_amdgcn_s_barrier();
        const uint8_t* Xs = smem + (ch & 1) * STAGE;
        const uint8_t* Ws_ = Xs + XB;
#pragma unroll
        for (int tap = 0; tap < KK; ++tap) {
            const int kh = tap / K, kw = tap - kh * K;
            bf16x8_t wf[2], xf[FN];
#pragma unroll
            for (int j = 0; j < 2; ++j)
                wf[j] = *reinterpret_cast<const bf16x8_t*>(Ws_ + (wrec[j] + tap) * kRec2 + wsw[j]);
#pragma unroll
            for (int i = 0; i < FN; ++i) {
                const int rec = pbase[i] + kh * PC + kw;
                xf[i] = *reinterpret_cast<const bf16x8_t*>(Xs + rec * kRec2 + ((g ^ ((rec >> kSwzBit) & 1)) << 4));
            }
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < FN; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j], xf[i], acc[j][i], 0, 0, 0);
        }
        // every wave's reads of this stage are done before it is refilled
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        if (ch + 2 < nch) issue((ch + 2) * kCi2, ch & 1);
    }

    // The stores go through LDS (ending in a barrier, so the statistics
    // below may reuse it).
    conv_store_lds<T, RES, FN>(a, acc, smem, co0, oh0, ow0, wco, wpx, lrow, g, e.lt, n);
    if constexpr (STATS) {
        float* red = reinterpret_cast<float*>(smem);
        switch (a.cg) {
            case 4: conv_group_stats_reg<T, 4, 4>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
            case 8: conv_group_stats_reg<T, 8, 4>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
            case 16: conv_group_stats_reg<T, 16, 4>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
            case 32: conv_group_stats_reg<T, 32, 4>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
            default: conv_group_stats_reg<T, 64, 4>(a, acc, red, co0, oh0, ow0, wco, wpx, lrow, g, wave); break;
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

namespace dit {
namespace {

// Tile geometry of an output image of Hs x Ws: TC = 128, 64, 32 or 16 columns.
void conv_geometry(int64_t Hs, int64_t Ws, int* TR, int* TC, int64_t* tiles_w, int64_t* tiles_h) {
    *TC = Ws >= 128 ? 128 : Ws >= 64 ? 64 : Ws >= 32 ? 32 : 16;
    *TR = kTilePx / *TC;
    *tiles_w = (Ws + *TC - 1) / *TC;
    *tiles_h = (Hs + *TR - 1) / *TR;
}

int64_t nhwc_elems(int64_t N, int64_t Ci, int64_t H, int64_t W) { return N * H * W * pad_to(Ci, kCi2); }

// Tile geometry of the DMA kernel: 256-pixel tiles, TC = 256 .. 16 columns.
// The DMA kernel's 256-pixel tile: 8 rows of 32 (16 x 16 on narrower
// images).  Its input patch is then 10 x 34 records against 3 x 258 for a
// 1 x 256 strip, and on gfx950 it ran 3-22% faster than the 1 x 256, 2 x 128
// and 4 x 64 tiles at every decoder shape ([1,128,1024,1024] -> 128 bf16:
// 784 / 760 / 765 us against 701 us, channel-last copy included), with the
// same output bits.
// px: the tile's pixels, 256 or 512 (16 x 32).
void conv_geometry2(int64_t Hs, int64_t Ws, int px, int* TR, int* TC, int64_t* tiles_w, int64_t* tiles_h) {
    *TC = Ws >= 32 ? 32 : 16;
    *TR = px / *TC;
    *tiles_w = (Ws + *TC - 1) / *TC;
    *tiles_h = (Hs + *TR - 1) / *TR;
}

// Launches the conv; with a workspace of dt_conv2d_workspace_bytes (and, for
// statistics, 4..64 channels per group) the transpose + DMA kernel, else the
// register-staged one.  *n_tiles: the pixel tiles of the launch.
int conv_launch(const void* x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void* packed_w, int64_t Co,
                int64_t K, int32_t upscale2, const float* bias, void* y, int32_t io_type, float4* stats,
                int64_t groups, const void* ws, size_t ws_bytes, hipStream_t st, const char* what,
                int64_t* n_tiles, const ConvFold* fold = nullptr) {
    const ConvFold none{};
    if (!fold) fold = &none;
    const int res_mode = fold->res_mode;
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
    a.stats = stats;
    a.G = (int)groups;
    a.cg = groups > 0 ? (int)(Co / groups) : 0;
    DT_REQUIRE(!res_mode || (fold->res && !stats), "%s: the residual epilogue needs a residual and no statistics",
               what);
    a.res = fold->res;
    a.res_mode = res_mode;
    a.res_scale = fold->res_scale;
    const bool gn = fold->gn_mr != nullptr;
    DT_REQUIRE(!gn || (fold->gn_groups > 0 && Ci % fold->gn_groups == 0 && !stats),
               "%s: the GroupNorm fold needs groups dividing the input channels", what);
    // With a workspace 3x3 convs, and 1x1 convs on bf16, take the DMA path
    // (gfx950, 1x1 [1, 256, 512, 512] -> 128: bf16 158 us against 217 us
    // staged; fp32 163 us against 136 us, its channel-last copy reading
    // twice the bytes).
    const bool dma = conv_uses_dma(K, io_type) && ws && ws_bytes >= (size_t)(nhwc_elems(N, Ci, H, W) * 2 + 256) &&
                     aligned16(ws) && (!stats || (a.cg >= 4 && a.cg <= 64));
    int64_t tiles_w, tiles_h;
    DT_REQUIRE(!gn || dma, "%s: the GroupNorm fold needs a 3x3 conv with a workspace", what);
    // 512-pixel tiles (half the weight DMA per output pixel) when they still
    // give two workgroups per CU; statistics and the residual epilogue keep
    // 256-pixel tiles (their registers would spill with 256 accumulators).
    int fn = 4;
    if (dma && !stats && !res_mode) {
        int tr, tc;
        int64_t tw, th;
        conv_geometry2(Hs, Ws, 512, &tr, &tc, &tw, &th);
        if (tw * th * ((Co + kTileCo - 1) / kTileCo) * N >= 512) fn = 8;
    }
    if (dma) conv_geometry2(Hs, Ws, 64 * fn, &a.TR, &a.TC, &tiles_w, &tiles_h);
    else conv_geometry(Hs, Ws, &a.TR, &a.TC, &tiles_w, &tiles_h);
    a.tiles_w = (int)tiles_w;
    DT_REQUIRE(tiles_h * tiles_w < (1ll << 31), "%s: too many tiles", what);
    *n_tiles = tiles_h * tiles_w;
    const dim3 grid((unsigned)(tiles_h * tiles_w), (unsigned)((Co + kTileCo - 1) / kTileCo), (unsigned)N);
    if (dma) {
        Conv2Extra e{};
        const int64_t elems = nhwc_elems(N, Ci, H, W);
        e.xh = (const uint16_t*)ws;
        e.zero = (const uint16_t*)ws + elems;
        e.C16 = (int)pad_to(Ci, kCi2);
        e.Cp32 = a.Ci_pad;
        e.lt = __builtin_ctz((unsigned)a.TC);
        const int64_t HW = H * W;
        const dim3 tg((unsigned)((HW + 63) / 64), (unsigned)((e.C16 + 63) / 64), (unsigned)N);
        const bool vec = HW % 8 == 0 && aligned16(x);
        const CopyGn cgn{fold->gn_mr, fold->gn_w, fold->gn_b, fold->gn_groups,
                         gn ? (int)(Ci / fold->gn_groups) : 1, fold->gn_silu};
#define DT_NHWC(TT, VV)                                                                                        \
    do {                                                                                                       \
        if (gn)                                                                                                \
            hipLaunchKernelGGL((to_nhwc16_kernel<TT, VV, true>), tg, dim3(256), 0, st, (const TT*)x, (int)Ci, HW, \
                               e.C16, (uint16_t*)ws, elems, cgn);                                              \
        else                                                                                                   \
            hipLaunchKernelGGL((to_nhwc16_kernel<TT, VV, false>), tg, dim3(256), 0, st, (const TT*)x, (int)Ci, HW, \
                               e.C16, (uint16_t*)ws, elems, cgn);                                              \
    } while (0)
        if (io_type == DT_TYPE_F32) {
            if (vec) DT_NHWC(float, true);
            else DT_NHWC(float, false);
        } else {
            if (vec) DT_NHWC(bf16, true);
            else DT_NHWC(bf16, false);
        }
#undef DT_NHWC
        int rc = check_launch(what);
        if (rc) return rc;
#define DT_CONV2_LAUNCH(TT, KS, ST, RS)                                                                     \
    do {                                                                                                    \
        if (fn == 8)                                                                                        \
            hipLaunchKernelGGL((conv2d_dma_kernel<TT, KS, ST, RS, ((ST || RS) ? 4 : 8)>), grid, dim3(256), 0, st, a, e); \
        else                                                                                                \
            hipLaunchKernelGGL((conv2d_dma_kernel<TT, KS, ST, RS, 4>), grid, dim3(256), 0, st, a, e);       \
    } while (0)
        if (io_type == DT_TYPE_F32) {
            if (K == 1) {
                if (stats) DT_CONV2_LAUNCH(float, 1, true, false);
                else if (res_mode) DT_CONV2_LAUNCH(float, 1, false, true);
                else DT_CONV2_LAUNCH(float, 1, false, false);
            } else {
                if (stats) DT_CONV2_LAUNCH(float, 3, true, false);
                else if (res_mode) DT_CONV2_LAUNCH(float, 3, false, true);
                else DT_CONV2_LAUNCH(float, 3, false, false);
            }
        } else {
            if (K == 1) {
                if (stats) DT_CONV2_LAUNCH(bf16, 1, true, false);
                else if (res_mode) DT_CONV2_LAUNCH(bf16, 1, false, true);
                else DT_CONV2_LAUNCH(bf16, 1, false, false);
            } else {
                if (stats) DT_CONV2_LAUNCH(bf16, 3, true, false);
                else if (res_mode) DT_CONV2_LAUNCH(bf16, 3, false, true);
                else DT_CONV2_LAUNCH(bf16, 3, false, false);
            }
        }
#undef DT_CONV2_LAUNCH
        return check_launch(what);
    }
#define DT_CONV_LAUNCH(TT, KS)                                                                         \
    do {                                                                                               \
        if (stats) hipLaunchKernelGGL((conv2d_kernel<TT, KS, true, false>), grid, dim3(256), 0, st, a);   \
        else if (res_mode) hipLaunchKernelGGL((conv2d_kernel<TT, KS, false, true>), grid, dim3(256), 0, st, a); \
        else hipLaunchKernelGGL((conv2d_kernel<TT, KS, false, false>), grid, dim3(256), 0, st, a);        \
    } while (0)
    if (io_type == DT_TYPE_F32) {
        if (K == 3) DT_CONV_LAUNCH(float, 3);
        else DT_CONV_LAUNCH(float, 1);
    } else {
        if (K == 3) DT_CONV_LAUNCH(bf16, 3);
        else DT_CONV_LAUNCH(bf16, 1);
    }
#undef DT_CONV_LAUNCH
    return check_launch(what);
}

}  // namespace
}  // namespace dit

extern "C" size_t dt_conv2d_workspace_bytes(int64_t N, int64_t Ci, int64_t H, int64_t W) {
    if (N <= 0 || Ci <= 0 || H <= 0 || W <= 0) return 0;
    return (size_t)(dit::nhwc_elems(N, Ci, H, W) * 2 + 256);
}

extern "C" int dt_conv2d(const void* x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void* packed_w,
                         int64_t Co, int64_t K, int32_t upscale2, const float* bias, void* y, void* workspace,
                         size_t workspace_bytes, int32_t io_type, dt_stream_t stream) {
    int64_t tiles;
    return dit::conv_launch(x, N, Ci, H, W, packed_w, Co, K, upscale2, bias, y, io_type, nullptr, 0, workspace,
                            workspace_bytes, (hipStream_t)stream, "dt_conv2d", &tiles);
}

namespace dit {

int conv2d_fold(const void* x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void* packed_w, int64_t Co,
                int64_t K, int32_t upscale2, const float* bias, const ConvFold& fold, void* y, void* workspace,
                size_t workspace_bytes, int32_t io_type, hipStream_t st) {
    int64_t tiles;
    return conv_launch(x, N, Ci, H, W, packed_w, Co, K, upscale2, bias, y, io_type, nullptr, 0, workspace,
                       workspace_bytes, st, "conv2d_fold", &tiles, &fold);
}

}  // namespace dit

extern "C" size_t dt_conv2d_gn_stats_bytes(int64_t N, int64_t Co, int64_t OH, int64_t OW, int64_t groups) {
    if (N <= 0 || Co <= 0 || OH <= 0 || OW <= 0 || groups <= 0 || Co % groups) return 0;
    int tr, tc;
    int64_t tw, th;
    dit::conv_geometry(OH, OW, &tr, &tc, &tw, &th);  // the finer tiling: enough records for either kernel
    return (size_t)(dit::gn_tile_stats_head_bytes(N, groups) + N * groups * th * tw * 16);
}

extern "C" int dt_conv2d_gn(const void* x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void* packed_w,
                            int64_t Co, int64_t K, int32_t upscale2, const float* bias, void* y, int64_t groups,
                            void* stats, size_t stats_bytes, void* workspace, size_t workspace_bytes,
                            int32_t io_type, dt_stream_t stream) {
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
    int64_t tiles;
    int rc = conv_launch(x, N, Ci, H, W, packed_w, Co, K, upscale2, bias, y, io_type, recs, groups, workspace,
                         workspace_bytes, st, "dt_conv2d_gn", &tiles);
    if (rc) return rc;
    return gn_tile_stats_finalize(stats, N, groups, tiles, st);
}

namespace dit {
namespace {

template <typename T>
__global__ void upscale_nearest_kernel(const T* __restrict__ x, int64_t H, int64_t W, int f, T* __restrict__ y,
                                       int64_t total) {
    const int64_t Wo = W * f, Ho = H * f;
    for (int64_t i = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; i < total; i += (int64_t)gridDim.x * blockDim.x) {
        const int64_t j = i % Wo, r = i / Wo, oi = r % Ho, plane = r / Ho;
        y[i] = x[(plane * H + oi / f) * W + j / f];
    }
}

}  // namespace
}  // namespace dit

extern "C" int dt_op_upscale_nearest(const void* src, int64_t N, int64_t C, int64_t H, int64_t W, int32_t factor,
                                     void* dst, int32_t io_type, dt_stream_t stream) {
    using namespace dit;
    DT_REQUIRE(is_io_type(io_type), "dt_op_upscale_nearest: io_type %d unsupported", io_type);
    DT_REQUIRE(N > 0 && C > 0 && H > 0 && W > 0 && factor >= 1, "dt_op_upscale_nearest: bad shape");
    DT_REQUIRE(src && dst, "dt_op_upscale_nearest: null pointer");
    const int64_t total = N * C * H * W * factor * factor;
    const unsigned grid = (unsigned)std::min<int64_t>((total + 255) / 256, 65536);
    if (io_type == DT_TYPE_F32)
        hipLaunchKernelGGL((upscale_nearest_kernel<float>), dim3(grid), dim3(256), 0, (hipStream_t)stream,
                           (const float*)src, H, W, factor, (float*)dst, total);
    else
        hipLaunchKernelGGL((upscale_nearest_kernel<uint16_t>), dim3(grid), dim3(256), 0, (hipStream_t)stream,
                           (const uint16_t*)src, H, W, factor, (uint16_t*)dst, total);
    return check_launch("dt_op_upscale_nearest");
}
