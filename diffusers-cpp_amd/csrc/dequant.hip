// dequant.hip -- ggml Q8_0 / Q4_K weight dequantisation to bf16 or fp32,
// bit-exact with ggml's dequantize_row_q8_0 / dequantize_row_q4_K.
//
// Work unit: one lane produces 8 consecutive outputs (one 16-byte bf16 store,
// two for fp32), so a wave writes 1 KB of contiguous output per instruction.
// Rows that are 16-byte aligned (every GGUF tensor; Q4_K always) are staged:
// a workgroup copies its run of blocks into LDS with 16-byte streaming loads
// (the 34-byte Q8_0 block has no wider alignment than 2 bytes, and the Q4_K
// header is shared by 32 lanes), then decodes from LDS.  Otherwise each lane
// gathers its block from global memory directly.
//   Q8_0  block = {fp16 d; int8 qs[32]} (34 B): 4 lanes share a block, each
//         reads d and 8 quant bytes (2-byte aligned -> four u16 loads).
//         d*q is exact in fp32 (11-bit x 8-bit significands).
//   Q4_K  super-block = {fp16 d, dmin; u8 scales[12]; u8 qs[128]} (144 B):
//         32 lanes share a super-block; each reads the 16-byte header and 8
//         quant bytes (one 16 B + one 8 B load), decodes its sub-block's
//         6-bit (scale, min) and computes (d*sc)*q - (dmin*m) with each
//         operation rounded separately.
#include "capi_util.hpp"
#include "common.hpp"

namespace dit {
namespace {

template <typename T>
__device__ __forceinline__ void store_out8(T* p, const float* v);
template <>
__device__ __forceinline__ void store_out8<bf16>(bf16* p, const float* v) { Io<bf16>::store(p, v); }
template <>
__device__ __forceinline__ void store_out8<float>(float* p, const float* v) {
    Io<float>::store(p, v);
    Io<float>::store(p + 4, v + 4);
}

// Lane `part` (0..3) of Q8_0 block h (fp16 d, then 32 int8 codes as 16
// halfwords): outputs [8 part, 8 part + 8) of the block, stored at out.
template <typename T>
__device__ __forceinline__ void q8_0_decode8(const uint16_t* h, uint32_t part, T* out) {
    const float d = f16_bits_to_f32(h[0]);
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t two = h[1 + part * 4 + i];
        v[2 * i] = mul_rn(d, (float)(int8_t)(two & 0xFF));
        v[2 * i + 1] = mul_rn(d, (float)(int8_t)(two >> 8));
    }
    store_out8<T>(out + part * 8, v);
}

// Lane k (0..31) of the Q4_K super-block at b: outputs [8k, 8k + 8), stored
// at out.  Sub-block j = 2*c64 + hi; header bytes 4..15 are scales[0..11].
template <typename T>
__device__ __forceinline__ void q4_K_decode8(const uint8_t* b, uint32_t k, T* out) {
    const uint32_t e0 = k * 8;                            // element offset in the super-block
    const uint32_t c64 = e0 >> 6, o = e0 & 63, hi = o >> 5, l0 = o & 31;
    const uint4 hdr = *reinterpret_cast<const uint4*>(b);
    const uint2 q8 = *reinterpret_cast<const uint2*>(b + 16 + 32 * c64 + l0);
    const uint32_t j = 2 * c64 + hi, sh = 8 * (j & 3);
    const uint32_t by = (hdr.y >> sh) & 0xFF;   // scales[j & 3]
    const uint32_t bz = (hdr.z >> sh) & 0xFF;   // scales[(j & 3) + 4]
    const uint32_t bw = (hdr.w >> sh) & 0xFF;   // scales[(j & 3) + 8]
    uint32_t sc, m;
    if (j < 4) {
        sc = by & 63;
        m = bz & 63;
    } else {
        sc = (bw & 0xF) | ((by >> 6) << 4);
        m = (bw >> 4) | ((bz >> 6) << 4);
    }
    const float d1 = mul_rn(f16_bits_to_f32(hdr.x & 0xFFFF), (float)sc);
    const float m1 = mul_rn(f16_bits_to_f32(hdr.x >> 16), (float)m);
    const uint32_t shift = hi * 4;
    float v[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[i] = sub_rn(mul_rn(d1, (float)((q8.x >> (8 * i + shift)) & 0xF)), m1);
        v[4 + i] = sub_rn(mul_rn(d1, (float)((q8.y >> (8 * i + shift)) & 0xF)), m1);
    }
    store_out8<T>(out + e0, v);
}

template <typename T>
__global__ __launch_bounds__(256) void dequant_q8_0_kernel(const uint8_t* __restrict__ src,
                                                           int64_t row_bytes, T* __restrict__ dst,
                                                           int64_t dst_stride, uint32_t total,
                                                           FastDiv chunks_per_row) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const uint32_t r = fdiv(idx, chunks_per_row);
    const uint32_t k = idx - r * chunks_per_row.d;
    const uint32_t blk = k >> 2, part = k & 3;
    const uint8_t* b = src + (int64_t)r * row_bytes + (int64_t)blk * 34;
    q8_0_decode8<T>(reinterpret_cast<const uint16_t*>(b), part, dst + (int64_t)r * dst_stride + (int64_t)blk * 32);
}

template <typename T>
__global__ __launch_bounds__(256) void dequant_q4_K_kernel(const uint8_t* __restrict__ src,
                                                           int64_t row_bytes, T* __restrict__ dst,
                                                           int64_t dst_stride, uint32_t total,
                                                           FastDiv chunks_per_row) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const uint32_t r = fdiv(idx, chunks_per_row);
    const uint32_t k = idx - r * chunks_per_row.d;
    const uint32_t blk = k >> 5;
    const uint8_t* b = src + (int64_t)r * row_bytes + (int64_t)blk * 144;   // header shared by 32 lanes: cached
    q4_K_decode8<T>(b, k & 31, dst + (int64_t)r * dst_stride + (int64_t)blk * 256);
}

constexpr int kStageThreads = 256;
constexpr int kQ8SegBlocks = kStageThreads / 4;   // 64 blocks = 2176 B = 136 x 16 B
constexpr int kQ4SegBlocks = kStageThreads / 32;  // 8 super-blocks = 1152 B = 72 x 16 B

// Q8_0, staged: workgroup (seg, row) decodes blocks [64 seg, 64 seg + 64) of
// the row.  64 blocks start at a multiple of 2176 bytes, so with 16-byte
// aligned rows the run starts aligned, and its rounded-up end stays inside
// the row (row_bytes is a multiple of 16 and at least 34 * blocks).
template <typename T>
__global__ __launch_bounds__(kStageThreads) void dequant_q8_0_staged_kernel(const uint8_t* __restrict__ src,
                                                                            int64_t row_bytes, T* __restrict__ dst,
                                                                            int64_t dst_stride, int blocks_per_row,
                                                                            int segs) {
    __shared__ __attribute__((aligned(16))) uint4 stage[kQ8SegBlocks * 34 / 16];
    const int row = blockIdx.x / segs, seg = blockIdx.x - row * segs, t = threadIdx.x;
    const int b0 = seg * kQ8SegBlocks, nblk = min(kQ8SegBlocks, blocks_per_row - b0);
    const uint8_t* base = src + (int64_t)row * row_bytes + (int64_t)b0 * 34;
    if (t < (nblk * 34 + 15) / 16) stage[t] = ld_stream(base + 16 * t);
    __syncthreads();
    const int blk = t >> 2, part = t & 3;
    if (blk >= nblk) return;
    q8_0_decode8<T>(reinterpret_cast<const uint16_t*>(stage) + blk * 17, part,
                    dst + (int64_t)row * dst_stride + (int64_t)(b0 + blk) * 32);
}

// Q4_K, staged: workgroup (seg, row) decodes super-blocks [8 seg, 8 seg + 8)
// of the row (144 B each, 16-byte aligned), 32 lanes per super-block.
template <typename T>
__global__ __launch_bounds__(kStageThreads) void dequant_q4_K_staged_kernel(const uint8_t* __restrict__ src,
                                                                            int64_t row_bytes, T* __restrict__ dst,
                                                                            int64_t dst_stride, int blocks_per_row,
                                                                            int segs) {
    __shared__ __attribute__((aligned(16))) uint4 stage[kQ4SegBlocks * 9];
    const int row = blockIdx.x / segs, seg = blockIdx.x - row * segs, t = threadIdx.x;
    const int b0 = seg * kQ4SegBlocks, nblk = min(kQ4SegBlocks, blocks_per_row - b0);
    const uint8_t* base = src + (int64_t)row * row_bytes + (int64_t)b0 * 144;
    if (t < nblk * 9) stage[t] = ld_stream(base + 16 * t);
    __syncthreads();
    const int sb = t >> 5, k = t & 31;
    if (sb >= nblk) return;
    q4_K_decode8<T>(reinterpret_cast<const uint8_t*>(stage) + sb * 144, k,
                    dst + (int64_t)row * dst_stride + (int64_t)(b0 + sb) * 256);
}

// Dense tensors (rows packed back to back in the source and the output) are
// one stream of blocks: workgroup i decodes blocks [SEG * i, SEG * i + SEG)
// with SEG = U x the staged kernels' run.  At U = 8 a workgroup keeps 17 KB
// (Q8_0) / 9 KB (Q4_K) of loads in flight, the fastest run for tensors that
// fill the chip (4x and 16x measured slower at 3072 x 9216); smaller tensors
// take a shorter run (flat_unroll).  The bytes past the last whole 16-byte
// vector of the tensor are copied in 2-byte pieces, so nothing past the
// tensor is read.
constexpr int kFlatUnroll = 8;

template <typename T, int U>
__global__ __launch_bounds__(kStageThreads) void dequant_q8_0_flat_kernel(const uint8_t* __restrict__ src,
                                                                          int64_t nblocks, T* __restrict__ dst) {
    constexpr int SEG = kQ8SegBlocks * U;
    __shared__ __attribute__((aligned(16))) uint4 stage[SEG * 34 / 16];
    const int t = threadIdx.x;
    const int64_t b0 = (int64_t)blockIdx.x * SEG;
    const int nblk = (int)min<int64_t>(SEG, nblocks - b0);
    const uint8_t* base = src + b0 * 34;
    const int bytes = nblk * 34, nvec = bytes >> 4;
    for (int i = t; i < nvec; i += kStageThreads) stage[i] = ld_stream(base + 16 * i);
    if (t < (bytes & 15) / 2)
        reinterpret_cast<uint16_t*>(stage)[nvec * 8 + t] = reinterpret_cast<const uint16_t*>(base + 16 * nvec)[t];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int blk = u * kQ8SegBlocks + (t >> 2);
        if (blk < nblk) q8_0_decode8<T>(reinterpret_cast<const uint16_t*>(stage) + blk * 17, t & 3, dst + (b0 + blk) * 32);
    }
}

template <typename T, int U>
__global__ __launch_bounds__(kStageThreads) void dequant_q4_K_flat_kernel(const uint8_t* __restrict__ src,
                                                                          int64_t nblocks, T* __restrict__ dst) {
    constexpr int SEG = kQ4SegBlocks * U;
    __shared__ __attribute__((aligned(16))) uint4 stage[SEG * 9];
    const int t = threadIdx.x;
    const int64_t b0 = (int64_t)blockIdx.x * SEG;
    const int nblk = (int)min<int64_t>(SEG, nblocks - b0);
    const uint8_t* base = src + b0 * 144;
    // streaming loads: default (cache-allocating) ones measured 3% faster back
    // to back at 3072 x 3072 but 14-21% slower as single launches after other
    // work filled the caches (3072 x 9216: 15.5 -> 18.8 us)
    for (int i = t; i < nblk * 9; i += kStageThreads) stage[i] = ld_stream(base + 16 * i);
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int sb = u * kQ4SegBlocks + (t >> 5);
        if (sb < nblk) q4_K_decode8<T>(reinterpret_cast<const uint8_t*>(stage) + sb * 144, t & 31, dst + (b0 + sb) * 256);
    }
}

// The same runs in two halves, for U = 2 and 4 (tensors that fill the chip
// in one round with shorter runs): every load of the run is issued at once,
// the first half is decoded and stored while the second half's loads are in
// flight, then the second half.  At 3072 x 3072 (U = 4) this took Q4_K from
// 5.36 to 4.83 us and Q8_0 from 6.20 to 5.83 us back to back, the same bits.
// At U = 8 it was slower (Q4_K 12.6 -> 14.3 us at 3072 x 9216; issuing the
// whole run's loads at once without the halves, 13.7 us): there the flat
// kernels' load loop, whose trips wait for each load before its LDS write,
// keeps fewer reads in flight and is the fastest form measured.
// A partial last run (nblocks not a multiple of the run) takes the flat
// kernels' path, uniformly for its workgroup.
template <typename T, int U>
__global__ __launch_bounds__(kStageThreads) void dequant_q8_0_halves_kernel(const uint8_t* __restrict__ src,
                                                                            int64_t nblocks, T* __restrict__ dst) {
    constexpr int SEG = kQ8SegBlocks * U, NVEC = SEG * 34 / 16, HV = NVEC / 2;
    constexpr int LH = (HV + kStageThreads - 1) / kStageThreads;      // loads per thread per half
    static_assert(SEG * 34 % 32 == 0, "each half is whole 16-byte vectors");
    __shared__ __attribute__((aligned(16))) uint4 stage[NVEC];
    const int t = threadIdx.x;
    const int64_t b0 = (int64_t)blockIdx.x * SEG;
    const int nblk = (int)min<int64_t>(SEG, nblocks - b0);
    const uint8_t* base = src + b0 * 34;
    const uint16_t* h = reinterpret_cast<const uint16_t*>(stage);
    if (nblk < SEG) {
        const int bytes = nblk * 34, nvec = bytes >> 4;
        for (int i = t; i < nvec; i += kStageThreads) stage[i] = ld_stream(base + 16 * i);
        if (t < (bytes & 15) / 2)
            reinterpret_cast<uint16_t*>(stage)[nvec * 8 + t] = reinterpret_cast<const uint16_t*>(base + 16 * nvec)[t];
        __syncthreads();
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int blk = u * kQ8SegBlocks + (t >> 2);
            if (blk < nblk) q8_0_decode8<T>(h + blk * 17, t & 3, dst + (b0 + blk) * 32);
        }
        return;
    }
    // Vector i of each half; threads past the half reload its last vector
    // (same address, same LDS word), so every load is unconditional.
    int iv[LH];
    uint4 ra[LH], rb[LH];
#pragma unroll
    for (int l = 0; l < LH; ++l) {
        iv[l] = min(l * kStageThreads + t, HV - 1);
        ra[l] = ld_stream(base + 16 * iv[l]);
    }
#pragma unroll
    for (int l = 0; l < LH; ++l) rb[l] = ld_stream(base + 16 * (HV + iv[l]));
#pragma unroll
    for (int l = 0; l < LH; ++l) stage[iv[l]] = ra[l];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U / 2; ++u) {                 // blocks [0, SEG/2): bytes [0, 16 HV)
        const int blk = u * kQ8SegBlocks + (t >> 2);
        q8_0_decode8<T>(h + blk * 17, t & 3, dst + (b0 + blk) * 32);
    }
#pragma unroll
    for (int l = 0; l < LH; ++l) stage[HV + iv[l]] = rb[l];
    __syncthreads();
#pragma unroll
    for (int u = U / 2; u < U; ++u) {
        const int blk = u * kQ8SegBlocks + (t >> 2);
        q8_0_decode8<T>(h + blk * 17, t & 3, dst + (b0 + blk) * 32);
    }
}

template <typename T, int U>
__global__ __launch_bounds__(kStageThreads) void dequant_q4_K_halves_kernel(const uint8_t* __restrict__ src,
                                                                            int64_t nblocks, T* __restrict__ dst) {
    constexpr int SEG = kQ4SegBlocks * U, HV = SEG * 9 / 2;
    constexpr int LH = (HV + kStageThreads - 1) / kStageThreads;
    __shared__ __attribute__((aligned(16))) uint4 stage[SEG * 9];
    const int t = threadIdx.x;
    const int64_t b0 = (int64_t)blockIdx.x * SEG;
    const int nblk = (int)min<int64_t>(SEG, nblocks - b0);
    const uint8_t* base = src + b0 * 144;
    const uint8_t* sbs = reinterpret_cast<const uint8_t*>(stage);
    if (nblk < SEG) {
        for (int i = t; i < nblk * 9; i += kStageThreads) stage[i] = ld_stream(base + 16 * i);
        __syncthreads();
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int sb = u * kQ4SegBlocks + (t >> 5);
            if (sb < nblk) q4_K_decode8<T>(sbs + sb * 144, t & 31, dst + (b0 + sb) * 256);
        }
        return;
    }
    int iv[LH];
    uint4 ra[LH], rb[LH];
#pragma unroll
    for (int l = 0; l < LH; ++l) {
        iv[l] = min(l * kStageThreads + t, HV - 1);
        ra[l] = ld_stream(base + 16 * iv[l]);
    }
#pragma unroll
    for (int l = 0; l < LH; ++l) rb[l] = ld_stream(base + 16 * (HV + iv[l]));
#pragma unroll
    for (int l = 0; l < LH; ++l) stage[iv[l]] = ra[l];
    __syncthreads();
#pragma unroll
    for (int u = 0; u < U / 2; ++u) {                 // super-blocks [0, SEG/2): vectors [0, HV)
        const int sb = u * kQ4SegBlocks + (t >> 5);
        q4_K_decode8<T>(sbs + sb * 144, t & 31, dst + (b0 + sb) * 256);
    }
#pragma unroll
    for (int l = 0; l < LH; ++l) stage[HV + iv[l]] = rb[l];
    __syncthreads();
#pragma unroll
    for (int u = U / 2; u < U; ++u) {
        const int sb = u * kQ4SegBlocks + (t >> 5);
        q4_K_decode8<T>(sbs + sb * 144, t & 31, dst + (b0 + sb) * 256);
    }
}

// Runs per workgroup of the flat kernels: the smallest unroll whose
// workgroups are all resident at once (8 workgroups of 4 waves per CU), so no
// CU starts a second round while others idle; a tensor too large for one
// round runs in rounds of kFlatUnroll.  Measured back to back on 3072 x 3072:
// U = 4 (1152 workgroups) 6.2 / 5.4 us against U = 8 (576, two or three per
// CU) 7.5 / 6.4 us for Q8_0 / Q4_K, and U = 2 (2304, a second round) slower
// again; on 3072 x 9216, U = 8 (1728) is the fastest.
constexpr int kFlatResidentPerCu = 8;

int flat_unroll(int64_t nblocks, int64_t seg_blocks) {
    const int64_t slots = (int64_t)cu_count() * kFlatResidentPerCu;
    for (int u = 1; u < kFlatUnroll; u *= 2)
        if ((nblocks + seg_blocks * u - 1) / (seg_blocks * u) <= slots) return u;
    return kFlatUnroll;
}

template <typename T, int U>
void launch_flat(bool q8, const void* src, int64_t nblocks, void* dst, hipStream_t st) {
    const int64_t seg = (q8 ? kQ8SegBlocks : kQ4SegBlocks) * U;
    const dim3 grid((unsigned)((nblocks + seg - 1) / seg));
    constexpr bool halves = U == 2 || U == 4;
    if (q8 && halves)
        hipLaunchKernelGGL((dequant_q8_0_halves_kernel<T, U>), grid, dim3(kStageThreads), 0, st,
                           (const uint8_t*)src, nblocks, (T*)dst);
    else if (q8)
        hipLaunchKernelGGL((dequant_q8_0_flat_kernel<T, U>), grid, dim3(kStageThreads), 0, st, (const uint8_t*)src,
                           nblocks, (T*)dst);
    else if (halves)
        hipLaunchKernelGGL((dequant_q4_K_halves_kernel<T, U>), grid, dim3(kStageThreads), 0, st,
                           (const uint8_t*)src, nblocks, (T*)dst);
    else
        hipLaunchKernelGGL((dequant_q4_K_flat_kernel<T, U>), grid, dim3(kStageThreads), 0, st, (const uint8_t*)src,
                           nblocks, (T*)dst);
}

template <typename T>
int run(const void* src, int32_t qtype, int64_t rows, int64_t cols, int64_t row_bytes, void* dst,
        int64_t dst_stride, hipStream_t st) {
    {
        const bool q8 = qtype == DT_TYPE_Q8_0;
        const int64_t qk = q8 ? 32 : 256, bsz = q8 ? 34 : 144, per = q8 ? kQ8SegBlocks : kQ4SegBlocks;
        const int64_t nblocks = rows * (cols / qk);
        if (aligned16(src) && row_bytes == cols / qk * bsz && dst_stride == cols && nblocks / per < (1ll << 31)) {
            switch (flat_unroll(nblocks, per)) {
                case 1: launch_flat<T, 1>(q8, src, nblocks, dst, st); break;
                case 2: launch_flat<T, 2>(q8, src, nblocks, dst, st); break;
                case 4: launch_flat<T, 4>(q8, src, nblocks, dst, st); break;
                default: launch_flat<T, kFlatUnroll>(q8, src, nblocks, dst, st); break;
            }
            return check_launch("dt_dequant");
        }
    }
    const int64_t qk = qtype == DT_TYPE_Q8_0 ? 32 : 256, per = qtype == DT_TYPE_Q8_0 ? kQ8SegBlocks : kQ4SegBlocks;
    const int64_t bpr = cols / qk, segs = (bpr + per - 1) / per;
    if (aligned16(src) && row_bytes % 16 == 0 && rows * segs < (1ll << 31)) {
        const dim3 grid((unsigned)(rows * segs));
        if (qtype == DT_TYPE_Q8_0)
            hipLaunchKernelGGL((dequant_q8_0_staged_kernel<T>), grid, dim3(kStageThreads), 0, st,
                               (const uint8_t*)src, row_bytes, (T*)dst, dst_stride, (int)bpr, (int)segs);
        else
            hipLaunchKernelGGL((dequant_q4_K_staged_kernel<T>), grid, dim3(kStageThreads), 0, st,
                               (const uint8_t*)src, row_bytes, (T*)dst, dst_stride, (int)bpr, (int)segs);
        return check_launch("dt_dequant");
    }
    const int64_t cpr = cols / 8, total = rows * cpr;
    DT_REQUIRE(total < (1ll << 31), "dt_dequant: %lld chunks exceed the 32-bit index range",
               (long long)total);
    const unsigned blocks = (unsigned)((total + 255) / 256);
    const FastDiv fd = make_fastdiv((uint32_t)cpr);
    if (qtype == DT_TYPE_Q8_0)
        hipLaunchKernelGGL((dequant_q8_0_kernel<T>), dim3(blocks), dim3(256), 0, st,
                           (const uint8_t*)src, row_bytes, (T*)dst, dst_stride, (uint32_t)total, fd);
    else
        hipLaunchKernelGGL((dequant_q4_K_kernel<T>), dim3(blocks), dim3(256), 0, st,
                           (const uint8_t*)src, row_bytes, (T*)dst, dst_stride, (uint32_t)total, fd);
    return check_launch("dt_dequant");
}

}  // namespace
}  // namespace dit

extern "C" int dt_dequant(const void* src, int32_t qtype, int64_t rows, int64_t cols,
                          int64_t row_bytes, void* dst, int64_t dst_stride, int32_t dst_type,
                          dt_stream_t stream) {
    DT_REQUIRE(qtype == DT_TYPE_Q8_0 || qtype == DT_TYPE_Q4_K, "dt_dequant: qtype %d unsupported",
               qtype);
    DT_REQUIRE(dst_type == DT_TYPE_F32 || dst_type == DT_TYPE_BF16,
               "dt_dequant: dst_type %d unsupported", dst_type);
    DT_REQUIRE(rows >= 0 && cols > 0, "dt_dequant: bad shape");
    const int64_t qk = qtype == DT_TYPE_Q8_0 ? 32 : 256, bsz = qtype == DT_TYPE_Q8_0 ? 34 : 144;
    DT_REQUIRE(cols % qk == 0, "dt_dequant: cols %lld not a multiple of the block size %lld",
               (long long)cols, (long long)qk);
    DT_REQUIRE(row_bytes >= cols / qk * bsz, "dt_dequant: row_bytes %lld < %lld",
               (long long)row_bytes, (long long)(cols / qk * bsz));
    DT_REQUIRE(dst_stride >= cols, "dt_dequant: dst_stride < cols");
    if (rows == 0) return DT_OK;
    DT_REQUIRE(src && dst, "dt_dequant: null pointer");
    const int epv = dst_type == DT_TYPE_BF16 ? 8 : 4;
    DT_REQUIRE(dit::aligned16(dst) && dst_stride % epv == 0,
               "dt_dequant: dst must be 16-byte aligned with a stride multiple of %d", epv);
    if (qtype == DT_TYPE_Q8_0)
        DT_REQUIRE((reinterpret_cast<uintptr_t>(src) & 1) == 0 && row_bytes % 2 == 0,
                   "dt_dequant: Q8_0 rows must be 2-byte aligned");
    else
        DT_REQUIRE(dit::aligned16(src) && row_bytes % 16 == 0,
                   "dt_dequant: Q4_K rows must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    if (dst_type == DT_TYPE_F32) return dit::run<float>(src, qtype, rows, cols, row_bytes, dst, dst_stride, st);
    return dit::run<dit::bf16>(src, qtype, rows, cols, row_bytes, dst, dst_stride, st);
}

// ---------------------------------------------------------------------------
// Q8_0 quantisation (ggml quantize_row_q8_0_ref): per block of 32,
// d = amax / 127, id = d ? 1 / d : 0, q_j = roundf(x_j * id), d stored as the
// RNE fp16 of d.  Four lanes share a block (8 values each); amax is combined
// across the quad with two xor shuffles.  Used to make Q8_0 weight bytes on
// the device (the reference reads them from GGUF files,
// src/ggml/GGUFLoaderVisitor.cpp:214-281).
// ---------------------------------------------------------------------------
namespace dit {
namespace {

__global__ __launch_bounds__(256) void quantize_q8_0_kernel(const float* __restrict__ src, int64_t src_stride,
                                                            uint8_t* __restrict__ dst, int64_t row_bytes,
                                                            uint32_t total, FastDiv quads_per_row) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    const bool live = idx < total;
    const uint32_t r = live ? fdiv(idx, quads_per_row) : 0;
    const uint32_t k = live ? idx - r * quads_per_row.d : 0;
    const uint32_t blk = k >> 2, part = k & 3;
    float v[8];
    if (live) {
        const float4* p = reinterpret_cast<const float4*>(src + (int64_t)r * src_stride + (int64_t)k * 8);
        const float4 a = p[0], b = p[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w;
        v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = 0.f;
    }
    float amax = 0.f;
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(v[j]));
    // lanes 4i..4i+3 hold one block (threads of a quad are consecutive)
    amax = fmaxf(amax, __shfl_xor(amax, 1));
    amax = fmaxf(amax, __shfl_xor(amax, 2));
    if (!live) return;
    const float d = amax / 127.0f;
    const float id = d != 0.0f ? 1.0f / d : 0.0f;
    uint8_t* b = dst + (int64_t)r * row_bytes + (int64_t)blk * 34;
    if (part == 0) *reinterpret_cast<uint16_t*>(b) = f32_to_f16_bits(d);
    uint16_t* qs = reinterpret_cast<uint16_t*>(b + 2 + 8 * part);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int lo = (int)roundf(v[2 * j] * id), hi = (int)roundf(v[2 * j + 1] * id);
        qs[j] = (uint16_t)((lo & 0xFF) | ((hi & 0xFF) << 8));
    }
}

// Q8_0 -> the split layout the Q8_0 GEMM reads: codes u = q + 128 as uint8
// [rows][ld_codes] (the +128 bias lets the GEMM convert a byte with one
// v_cvt_f32_ubyte), and the block scales as fp32 transposed,
// scales[blk * ld_scales + row], so the scales of one k-block for a run of
// rows are contiguous.  One thread per block of 32.
__global__ __launch_bounds__(256) void q8_0_split_kernel(const uint8_t* __restrict__ src, int64_t row_bytes,
                                                         uint8_t* __restrict__ codes, int64_t ld_codes,
                                                         float* __restrict__ scales, int64_t ld_scales,
                                                         uint32_t total, FastDiv blocks_per_row) {
    const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
    if (idx >= total) return;
    const uint32_t r = fdiv(idx, blocks_per_row);
    const uint32_t blk = idx - r * blocks_per_row.d;
    const uint16_t* h = reinterpret_cast<const uint16_t*>(src + (int64_t)r * row_bytes + (int64_t)blk * 34);
    uint32_t w[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t lo = h[1 + 2 * i], hi = h[2 + 2 * i];
        w[i] = (lo | (hi << 16)) ^ 0x80808080u;  // int8 q -> uint8 q + 128, per byte
    }
    uint4* out = reinterpret_cast<uint4*>(codes + (int64_t)r * ld_codes + (int64_t)blk * 32);
    out[0] = make_uint4(w[0], w[1], w[2], w[3]);
    out[1] = make_uint4(w[4], w[5], w[6], w[7]);
    scales[(int64_t)blk * ld_scales + r] = f16_bits_to_f32(h[0]);
}

}  // namespace

}  // namespace dit

extern "C" int dt_q8_0_split(const void* src, int64_t rows, int64_t cols, int64_t row_bytes, void* codes,
                             int64_t ld_codes, float* scales, int64_t ld_scales, dt_stream_t stream) {
    DT_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, "dt_q8_0_split: cols %lld must be a positive multiple of 32",
               (long long)cols);
    DT_REQUIRE(row_bytes >= cols / 32 * 34 && row_bytes % 2 == 0, "dt_q8_0_split: bad row_bytes %lld",
               (long long)row_bytes);
    DT_REQUIRE(ld_codes >= cols && ld_codes % 16 == 0, "dt_q8_0_split: ld_codes must be >= cols and a multiple of 16");
    DT_REQUIRE(ld_scales >= rows, "dt_q8_0_split: ld_scales < rows");
    if (rows == 0) return DT_OK;
    DT_REQUIRE(src && codes && scales, "dt_q8_0_split: null pointer");
    DT_REQUIRE((reinterpret_cast<uintptr_t>(src) & 1) == 0 && dit::aligned16(codes),
               "dt_q8_0_split: src must be 2-byte and codes 16-byte aligned");
    const int64_t total = rows * (cols / 32);
    // the row of a block comes from fdiv, which is exact for numerators below 2^31
    DT_REQUIRE(total < (1ll << 31), "dt_q8_0_split: %lld blocks exceed the 2^31 limit", (long long)total);
    hipLaunchKernelGGL(dit::q8_0_split_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                       (hipStream_t)stream, (const uint8_t*)src, row_bytes, (uint8_t*)codes, ld_codes, scales,
                       ld_scales, (uint32_t)total, dit::make_fastdiv((uint32_t)(cols / 32)));
    return dit::check_launch("dt_q8_0_split");
}

extern "C" int64_t dt_q8_0_split_scale_offset(int64_t rows, int64_t cols) { return (rows * cols + 255) / 256 * 256; }

extern "C" int64_t dt_q8_0_split_bytes(int64_t rows, int64_t cols) {
    return dt_q8_0_split_scale_offset(rows, cols) + cols / 32 * rows * 4;
}

extern "C" int dt_quantize_q8_0(const float* src, int64_t rows, int64_t cols, int64_t src_stride, void* dst,
                                int64_t row_bytes, dt_stream_t stream) {
    DT_REQUIRE(rows >= 0 && cols > 0 && cols % 32 == 0, "dt_quantize_q8_0: cols must be a positive multiple of 32");
    DT_REQUIRE(src_stride >= cols && src_stride % 4 == 0, "dt_quantize_q8_0: bad src_stride");
    DT_REQUIRE(row_bytes >= cols / 32 * 34 && row_bytes % 2 == 0, "dt_quantize_q8_0: bad row_bytes");
    if (rows == 0) return DT_OK;
    DT_REQUIRE(src && dst, "dt_quantize_q8_0: null pointer");
    DT_REQUIRE(dit::aligned16(src) && (reinterpret_cast<uintptr_t>(dst) & 1) == 0,
               "dt_quantize_q8_0: src must be 16-byte and dst 2-byte aligned");
    const int64_t quads = cols / 8, total = rows * quads;
    DT_REQUIRE(total < (1ll << 31), "dt_quantize_q8_0: too many elements for one launch");
    const dit::FastDiv fd = dit::make_fastdiv((uint32_t)quads);
    const unsigned grid = (unsigned)((total + 255) / 256);
    hipLaunchKernelGGL(dit::quantize_q8_0_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, src, src_stride,
                       (uint8_t*)dst, row_bytes, (uint32_t)total, fd);
    return dit::check_launch("dt_quantize_q8_0");
}
