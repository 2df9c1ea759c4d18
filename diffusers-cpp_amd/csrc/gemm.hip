// gemm.hip -- bf16 MFMA GEMM for the Linear layers of a full denoising step
// (Linear::forward -> Runtime::mul_mat, src/nn/Linear.cpp:17-36):
//   C[m, n] = sum_k A[m, k] * B[n, k]  (+ bias[n]) (+ D[m, n]),  fp32 accumulation,
// with A = activations [M, K] and B = a Linear weight [N, K] (PyTorch's
// [out, in]), both K-contiguous, so 16-byte chunks along K are exactly the
// 8-element bf16 operands of v_mfma_f32_32x32x16_bf16.
//
// Tiling (gfx950): a 256-thread workgroup owns a 128x128 C tile; each wave
// owns 64x64 = 2x2 MFMA 32x32 tiles (64 fp32 accumulators per lane).  K
// advances 64 at a time: the next A/B tiles are fetched into registers while
// the MFMAs consume the current tiles from LDS (rows padded to 144 bytes so
// 8-lane 16-byte reads hit distinct banks).  Operand layout of the 32x32x16
// instruction: lane l supplies A[l % 32][8 (l / 32) + e] and
// B[8 (l / 32) + e][l % 32]; accumulator element i of lane l is
// C[8 (i / 4) + 4 (l / 32) + i % 4][l % 32].
#include "capi_util.hpp"
#include "common.hpp"

namespace dit {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int BM = 128, BN = 128, BK = 64;
constexpr int LDSW = BK + 8;  // padded LDS row, in bf16 elements

template <typename TC>
__device__ __forceinline__ void store_c(TC* p, float v);
template <>
__device__ __forceinline__ void store_c<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store_c<bf16>(bf16* p, float v) { p->bits = (uint16_t)f32_to_bf16_bits(v); }
__device__ __forceinline__ float load_c(const float* p) { return *p; }
__device__ __forceinline__ float load_c(const bf16* p) { return __uint_as_float((uint32_t)p->bits << 16); }

template <typename TC>
__global__ __launch_bounds__(256) void gemm_bf16_nt_kernel(const uint16_t* __restrict__ A, int64_t lda,
                                                           const uint16_t* __restrict__ B, int64_t ldb,
                                                           TC* C, int64_t ldc, int M, int N, int K,
                                                           const float* __restrict__ bias, const TC* Dm,
                                                           int64_t ldd) {
    __shared__ __attribute__((aligned(16))) uint16_t As[BM * LDSW];
    __shared__ __attribute__((aligned(16))) uint16_t Bs[BN * LDSW];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int tile_m = blockIdx.y * BM, tile_n = blockIdx.x * BN;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    // Global -> register mapping: chunk c = tid + 256 r covers row c / 8,
    // k-chunk c % 8 (8 bf16 = 16 bytes) of a 128 x 64 tile.
    uint4 ra[4], rb[4];
    auto load_tiles = [&](int k0) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int c = tid + 256 * r, row = c >> 3, kc = c & 7;
            const int gm = tile_m + row, gn = tile_n + row;
            ra[r] = gm < M ? *reinterpret_cast<const uint4*>(A + (int64_t)gm * lda + k0 + kc * 8)
                           : make_uint4(0, 0, 0, 0);
            rb[r] = gn < N ? *reinterpret_cast<const uint4*>(B + (int64_t)gn * ldb + k0 + kc * 8)
                           : make_uint4(0, 0, 0, 0);
        }
    };
    auto store_tiles = [&]() {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int c = tid + 256 * r, row = c >> 3, kc = c & 7;
            *reinterpret_cast<uint4*>(&As[row * LDSW + kc * 8]) = ra[r];
            *reinterpret_cast<uint4*>(&Bs[row * LDSW + kc * 8]) = rb[r];
        }
    };

    f32x16_t acc[2][2];
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[i][j][e] = 0.f;

    load_tiles(0);
    store_tiles();
    __syncthreads();
    const int lrow = lane & 31, lk = (lane >> 5) * 8;
    for (int k0 = 0; k0 < K; k0 += BK) {
        const bool more = k0 + BK < K;
        if (more) load_tiles(k0 + BK);  // in flight while the MFMAs run
#pragma unroll
        for (int kk = 0; kk < BK; kk += 16) {
            bf16x8_t af[2], bfr[2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
                af[i] = *reinterpret_cast<const bf16x8_t*>(&As[(wm + 32 * i + lrow) * LDSW + kk + lk]);
#pragma unroll
            for (int j = 0; j < 2; ++j)
                bfr[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[(wn + 32 * j + lrow) * LDSW + kk + lk]);
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[i][j], 0, 0, 0);
        }
        __syncthreads();
        if (more) {
            store_tiles();
            __syncthreads();
        }
    }

#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int col = tile_n + wn + 32 * j + lrow;
            if (col >= N) continue;
            const float bv = bias ? bias[col] : 0.f;
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                const int row = tile_m + wm + 32 * i + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
                if (row < M) {
                    float v = acc[i][j][e] + bv;
                    if (Dm) v += load_c(Dm + (int64_t)row * ldd + col);
                    store_c<TC>(C + (int64_t)row * ldc + col, v);
                }
            }
        }
    }
}

}  // namespace
}  // namespace dit

extern "C" int dt_gemm_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                            int64_t M, int64_t N, int64_t K, const float* bias, const void* addend,
                            int64_t ldd, int32_t c_type, dt_stream_t stream) {
    DT_REQUIRE(c_type == DT_TYPE_BF16 || c_type == DT_TYPE_F32, "dt_gemm_bf16: c_type %d unsupported",
               c_type);
    DT_REQUIRE(M >= 0 && N >= 0 && K > 0, "dt_gemm_bf16: bad shape");
    DT_REQUIRE(K % dit::BK == 0, "dt_gemm_bf16: K (%lld) must be a multiple of %d", (long long)K, dit::BK);
    DT_REQUIRE(lda >= K && ldb >= K && ldc >= N && lda % 8 == 0 && ldb % 8 == 0,
               "dt_gemm_bf16: leading dimensions must cover the rows and keep 16-byte alignment");
    DT_REQUIRE(!addend || ldd >= N, "dt_gemm_bf16: ldd < N");
    DT_REQUIRE(M < (1ll << 31) && N < (1ll << 31) && K < (1ll << 31), "dt_gemm_bf16: shape too large");
    if (M == 0 || N == 0) return DT_OK;
    DT_REQUIRE(A && B && C, "dt_gemm_bf16: null pointer");
    DT_REQUIRE(dit::aligned16(A) && dit::aligned16(B), "dt_gemm_bf16: A and B must be 16-byte aligned");
    const dim3 grid((unsigned)((N + dit::BN - 1) / dit::BN), (unsigned)((M + dit::BM - 1) / dit::BM));
    DT_REQUIRE(grid.y < 65536, "dt_gemm_bf16: M too large for one launch");
    hipStream_t st = (hipStream_t)stream;
    if (c_type == DT_TYPE_F32)
        hipLaunchKernelGGL((dit::gemm_bf16_nt_kernel<float>), grid, dim3(256), 0, st, (const uint16_t*)A, lda,
                           (const uint16_t*)B, ldb, (float*)C, ldc, (int)M, (int)N, (int)K, bias,
                           (const float*)addend, ldd);
    else
        hipLaunchKernelGGL((dit::gemm_bf16_nt_kernel<dit::bf16>), grid, dim3(256), 0, st, (const uint16_t*)A,
                           lda, (const uint16_t*)B, ldb, (dit::bf16*)C, ldc, (int)M, (int)N, (int)K,
                           bias, (const dit::bf16*)addend, ldd);
    return dit::check_launch("dt_gemm_bf16");
}
