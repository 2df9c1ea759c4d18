// gemm.hip -- bf16 MFMA GEMM for the Linear layers of a full denoising step
// (Linear::forward -> Runtime::mul_mat, src/nn/Linear.cpp:17-36):
//   C[m, n] = sum_k A[m, k] * B[n, k]  (+ bias[n]) (+ D[m, n]),  fp32 accumulation,
// with A = activations [M, K] and B = a Linear weight [N, K] (PyTorch's
// [out, in]), both K-contiguous, so 16-byte chunks along K are exactly the
// 8-element bf16 operands of v_mfma_f32_32x32x16_bf16.  One launch can run a
// group of up to kMaxGroup independent GEMMs (the q/k/v/gate/up projections
// of a block), whose tiles share the grid: no wave of workgroups is left
// half-empty at the end of each small GEMM.
//
// Three tile configurations (gfx950):
//  * 256 x 256, 8 waves of 128 x 64: A and B travel global -> LDS by direct
//    DMA (global_load_lds_dwordx4: lane i of an instruction writes its 16
//    bytes to LDS base + 16 i) through four stages of K = 32, so the loads for
//    k-tile kt + 3 are in flight while k-tile kt is multiplied and no
//    registers are spent on staging.  A stage row is 64 bytes (4 chunks of 8
//    bf16); chunk c of row r is stored at chunk c ^ swz(r), swz(r) =
//    ((r >> 1) ^ (r >> 2)) & 3, which makes the 16-byte reads of 8 (32-bank)
//    or 16 (64-bank) consecutive rows at one logical chunk hit distinct banks.
//  * 256 x 256, 4 waves of 128 x 128, two stages of K = 64: whole 128-byte
//    rows per DMA segment and operand reads software-pipelined one k-step
//    ahead; chosen for long K.
//  * 128 x 128, 4 waves of 64 x 64, two workgroups per CU: K = 64 per step
//    through two register-staged LDS stages (rows padded to 144 bytes), for
//    GEMMs too small to fill the CUs with 256 x 256 tiles.
//
// The MFMA computes the transposed tile C^T = B A^T: the weight rows are the
// instruction's A operand and the activation rows its B operand, so the
// accumulator element i of lane l is C[m = 32 fm + l % 32][n = 32 fn +
// 8 (i / 4) + 4 (l / 32) + i % 4] and every lane stores 4 consecutive n.
// Operand layout of the 32x32x16 instruction: lane l supplies
// A[l % 32][8 (l / 32) + e] and B[8 (l / 32) + e][l % 32].
//
// Workgroups are renumbered so that each XCD (8 per MI355X, one L2 each)
// runs its own runs of 4 consecutive tiles, and each GEMM's tiles are ordered in
// groups of GROUP_M tile rows so concurrently running tiles share A rows and
// B columns.  Rows past M or N load a clamped valid row: their products only
// reach C entries that are never stored.
#include <initializer_list>
#include <type_traits>

#include "capi_util.hpp"
#include "common.hpp"

namespace dit {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

// Tile rows per group: the whole 1024^2 step (bf16 weights, one HIP graph)
// measured 41.2-41.3 ms at 2 against 41.6-41.7 at 4, 41.5-41.6 at 1, 41.8 at
// 3 and 42.0 at 8 (same box, same bits).
constexpr int GROUP_M = 2;
constexpr int kMaxGroup = 8;

struct Problem {
    const uint16_t* A;
    const uint16_t* B;
    void* C;
    const void* D;
    const float* bias;
    int64_t lda, ldb, ldc, ldd;
    int M, N, K;
    // Q8_0 weights (split layout): B holds biased uint8 codes [N][ldb bytes],
    // Bs the fp32 block scales transposed, Bs[blk * ldbs + n]; null for bf16 B.
    const float* Bs;
    int64_t ldbs;
};

struct Group {
    Problem p[kMaxGroup];
    int tile_start[kMaxGroup + 1];  // prefix sums of each problem's tile count
    int count;
};

template <typename TC>
__device__ __forceinline__ void store4(TC* p, const float* v);
template <>
__device__ __forceinline__ void store4<float>(float* p, const float* v) {
    *reinterpret_cast<float4*>(p) = make_float4(v[0], v[1], v[2], v[3]);
}
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, const float* v) {
    *reinterpret_cast<uint2*>(p) = make_uint2(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]));
}
__device__ __forceinline__ float load_c(const float* p) { return *p; }
__device__ __forceinline__ float load_c(const bf16* p) { return __uint_as_float((uint32_t)p->bits << 16); }
template <typename TC>
__device__ __forceinline__ void store1(TC* p, float v);
template <>
__device__ __forceinline__ void store1<float>(float* p, float v) { *p = v; }
template <>
__device__ __forceinline__ void store1<bf16>(bf16* p, float v) { p->bits = (uint16_t)f32_to_bf16_bits(v); }

// Problem and tile of this workgroup.  The hardware hands workgroup b to XCD
// b % 8; it takes tile ((j / 4) * 8 + b % 8) * 4 + j % 4 (j = b / 8), so each
// XCD works through runs of 4 consecutive tiles (two 2-row tile columns of a
// group) spread across the grid -- over the whole step on one box 39.5-39.7
// ms (bf16 weights) against 39.8-40.0 ms with one contiguous range of tiles
// per XCD, which is kept when the count per XCD is not a multiple of 4.
// Then GROUP_M-row groups inside the problem.
template <int BM, int BN>
__device__ __forceinline__ const Problem& locate(const Group& g, int* tm, int* tn) {
    uint32_t bid = blockIdx.x;
    const uint32_t nb = gridDim.x, q = nb >> 3;
    if (bid < (q << 3)) {
        const uint32_t x = bid & 7u, j = bid >> 3;
        bid = (q & 3u) == 0 ? ((j >> 2) * 8 + x) * 4 + (j & 3u) : x * q + j;
    }
    int pi = 0;
    while (pi + 1 < g.count && (int)bid >= g.tile_start[pi + 1]) ++pi;
    const Problem& p = g.p[pi];
    const int local = (int)bid - g.tile_start[pi];
    const int tiles_m = (p.M + BM - 1) / BM, tiles_n = (p.N + BN - 1) / BN;
    const int per_group = GROUP_M * tiles_n;
    const int group = local / per_group, first_m = group * GROUP_M;
    const int rows = min(tiles_m - first_m, GROUP_M);
    const int in_group = local - group * per_group;
    *tm = first_m + in_group % rows;
    *tn = in_group / rows;
    return p;
}

// Bias / addend epilogue and store of one wave's FM x FN blocks of 32 x 32.
template <int FM, int FN, typename TC>
__device__ __forceinline__ void epilogue(const Problem& p, const f32x16_t (&acc)[FN][FM], int mw, int nw,
                                         int lane) {
    TC* C = reinterpret_cast<TC*>(p.C);
    const TC* Dm = reinterpret_cast<const TC*>(p.D);
    const int lrow = lane & 31, g = lane >> 5;
    const bool vec = (p.N % 4) == 0;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int m = mw + 32 * i + lrow;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = nw + 32 * j + 8 * q + 4 * g;
                if (n >= p.N) continue;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    v[e] = acc[j][i][4 * q + e];
                    if (p.bias && n + e < p.N) v[e] += p.bias[n + e];
                    if (Dm && n + e < p.N) v[e] += load_c(Dm + (int64_t)m * p.ldd + n + e);
                }
                TC* dst = C + (int64_t)m * p.ldc + n;
                if (vec && n + 4 <= p.N) {
                    store4<TC>(dst, v);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < p.N) store1<TC>(dst + e, v[e]);
                }
            }
        }
    }
}

// ---- 256 x 256, direct global -> LDS, 4 stages ------------------------------
constexpr int DBK = 32, DSTAGES = 4, DROWB = DBK * 2, DOPB = 256 * DROWB, DSTAGEB = 2 * DOPB;

__device__ __forceinline__ int swz(int r) { return ((r >> 1) ^ (r >> 2)) & 3; }

template <int N_OUT>
__device__ __forceinline__ void wait_vm() {
    // s_waitcnt vmcnt(N_OUT) with expcnt / lgkmcnt left at their maxima.
    __builtin_amdgcn_s_waitcnt((N_OUT & 15) | ((N_OUT >> 4) << 14) | 0x0F70);
}

template <typename TC>
__global__ __launch_bounds__(512) void gemm_dma256_kernel(const Group grp) {
    constexpr int FM = 4, FN = 2;  // wave sub-tile 128 (m) x 64 (n)
    __shared__ __attribute__((aligned(16))) uint8_t smem[DSTAGES * DSTAGEB];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tm, tn;
    const Problem& p = locate<256, 256>(grp, &tm, &tn);
    const int m0 = tm * 256, n0 = tn * 256;
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;

    // DMA sources: wave w fills rows [32 w, 32 w + 32) of both operands, two
    // instructions of 16 rows each; lane i covers row + i / 4, stored chunk i % 4.
    const uint16_t* ga[2];
    const uint16_t* gb[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int row = 32 * wave + 16 * j + (lane >> 2);
        const int c = (lane & 3) ^ swz(row);
        ga[j] = p.A + (int64_t)min(m0 + row, p.M - 1) * p.lda + c * 8;
        gb[j] = p.B + (int64_t)min(n0 + row, p.N - 1) * p.ldb + c * 8;
    }
    auto issue = [&](int kt, int s) {
        uint8_t* base = smem + s * DSTAGEB + 32 * wave * DROWB;
        const int k0 = kt * DBK;
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            __builtin_amdgcn_global_load_lds(ga[j] + k0, base + 16 * j * DROWB, 16, 0, 0);
            __builtin_amdgcn_global_load_lds(gb[j] + k0, base + DOPB + 16 * j * DROWB, 16, 0, 0);
        }
    };

    f32x16_t acc[FN][FM];
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.f;

    const int lrow = lane & 31, g = lane >> 5, sw = swz(lrow);
    const int nk = p.K / DBK;
#pragma unroll
    for (int s = 0; s < DSTAGES - 1; ++s)
        if (s < nk) issue(s, s);
    for (int kt = 0; kt < nk; ++kt) {
        const int ahead = min(nk - 1 - kt, DSTAGES - 2);
        if (ahead >= 2) wait_vm<8>();
        else if (ahead == 1) wait_vm<4>();
        else wait_vm<0>();
        // A bare barrier: the wait above already covers this wave's DMA into
        // stage kt, and no LDS is written by ds_write in this loop, so the
        // workgroup fence of __syncthreads (which would drain every DMA in
        // flight, vmcnt(0)) is not needed.  Each wave's ds_reads of the stage
        // reused next have returned (the MFMAs consumed them) before it arrives.
        __builtin_amdgcn_s_barrier();
        if (kt + DSTAGES - 1 < nk) issue(kt + DSTAGES - 1, (kt + DSTAGES - 1) % DSTAGES);
        const uint8_t* As = smem + (kt % DSTAGES) * DSTAGEB;
        const uint8_t* Bs = As + DOPB;
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
            const int pc = ((2 * kk + g) ^ sw) * 16;
            bf16x8_t wf[FN], xf[FM];
#pragma unroll
            for (int j = 0; j < FN; ++j)
                wf[j] = *reinterpret_cast<const bf16x8_t*>(Bs + (wn + 32 * j + lrow) * DROWB + pc);
#pragma unroll
            for (int i = 0; i < FM; ++i)
                xf[i] = *reinterpret_cast<const bf16x8_t*>(As + (wm + 32 * i + lrow) * DROWB + pc);
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int i = 0; i < FM; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j], xf[i], acc[j][i], 0, 0, 0);
        }
    }
    epilogue<FM, FN, TC>(p, acc, m0 + wm, n0 + wn, lane);
}

// ---- BM x 256, 4 or 8 waves, K = 64 per stage, 2 stages --------------------
// BM = 256, NW = 4: each wave owns a 128 x 128 quarter of the tile (4 x 4
// blocks of 32 x 32, 256 fp32 accumulators, one wave per SIMD): per k-step it
// reads 8 operands for 16 MFMAs.
// BM = 256, NW = 8 (the default for the step's products): each wave owns
// 128 x 64 (4 x 2 blocks, 128 accumulators, 208 VGPRs, two waves per SIMD),
// reading 6 operands for 8 MFMAs -- 1.5x the LDS reads per MFMA, but while
// one wave of a SIMD waits on its LDS reads, the stage DMA or the barrier,
// the other issues MFMAs.  Measured on gfx950 with the same stages and bits:
// 12-21% faster on every product of the step (4608 x 27648 x 3072: 865 ->
// 713 us, 1.10 PFLOP/s; 4096 x 4096 x 24576: 1.11 -> 1.24 PFLOP/s), and
// 14-18% with Q8_0 weights staged.
// BM = 224 (7 blocks of 32): the four waves side by side along n, each
// 224 x 64 (7 x 2 blocks, 224 accumulators, 9 operand reads for 14 MFMAs).
// M = 4608 then makes 21 tile rows, so a 4608 x 3072 product is 252 tiles on
// the 256 CUs instead of 216 256 x 256 tiles (16% of the CUs idle).
// Rows of 64 bf16 = 128 bytes per stage, so each DMA row segment is one whole
// L2 line (the 64-byte segments of K = 32 stages issue twice the requests and
// feed LDS at ~14 TB/s against ~22 TB/s with full lines, measured on gfx950
// for this tile shape).  Two stages of (BM + 256) x 128 bytes; chunk c of row
// r is stored at chunk c ^ swz8(r), swz8(r) = (r ^ (r >> 3)) & 7, so the
// 16-byte reads of 8 (32-bank) or 16 (64-bank) consecutive rows at one
// logical chunk hit distinct banks.  Operand reads are software-pipelined one
// k-step ahead.
constexpr int EBK = 64, EROWB = EBK * 2;

__device__ __forceinline__ int swz8(int r) { return (r ^ (r >> 3)) & 7; }

// SCHED: the next k-step's operand reads are interleaved one by one into the
// current step's MFMAs, and the stage DMA one instruction per MFMA after the
// barrier (sched_group_barrier), so the compiler keeps both operand sets
// live instead of reading each fragment just before its MFMAs with an LDS
// round trip exposed.
// Q8: the weight operand is Q8_0 in the split layout (uint8 codes u = q + 128
// [N][K] and fp32 block scales [K/32][N]).  Its codes and scales for k-tile
// kt + 2 are loaded into registers where the bf16 kernel issues their DMA
// (16 codes of 4 rows per thread), converted one k-tile later, w = fma(u, d,
// -128 d) = d * q (exact) rounded to bf16 -- the value dt_dequant writes --
// and written to the stage in the bf16 layout before the barrier that
// publishes it.  The MFMA sequence is then the bf16 kernel's: C equals
// dt_dequant followed by the bf16 GEMM bit for bit.  Each code is converted
// once per workgroup (the eight-wave gemm_q8_kernel converts each twice, after
// the LDS read); measured 4-16% faster than it on the step's products.
template <typename TC, bool SCHED, int BM, bool Q8 = false, int NW = 4>
__global__ __launch_bounds__(64 * NW) void gemm_k64_kernel(const Group grp) {
    static_assert(BM == 256 || BM == 224, "tile height");
    static_assert(NW == 4 || (NW == 8 && BM == 256), "eight waves: 256-row tiles");
    constexpr int WAVES_M = BM == 256 ? 2 : 1, WAVES_N = NW / WAVES_M;
    constexpr int FM = BM / WAVES_M / 32, FN = 256 / WAVES_N / 32;
    constexpr int AOPB = BM * EROWB, STAGEB = AOPB + 256 * EROWB, NS = 2;
    constexpr int A_DMA = BM / NW / 8;  // A rows per wave / 8 rows per DMA instruction
    constexpr int B_DMA = 256 / NW / 8;
    __shared__ __attribute__((aligned(16))) uint8_t smem[NS * STAGEB];

    const int tid = threadIdx.x, lane = tid & 63;
    // The wave index is uniform: read it into a scalar so every LDS
    // destination below is a scalar (M0 without a per-instruction
    // readfirstlane).
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tm, tn;
    const Problem& p = locate<BM, 256>(grp, &tm, &tn);
    const int m0 = tm * BM, n0 = tn * 256;
    const int wm = (wave / WAVES_N) * (BM / WAVES_M), wn = (wave % WAVES_N) * (256 / WAVES_N);

    // DMA sources: wave w fills A rows [BM/NW w, +BM/NW) and B rows
    // [256/NW w, +256/NW), instructions of 8 rows each; lane i covers row +
    // i / 8, stored chunk i % 8.  Buffer loads to LDS: the tile's first row is the
    // (scalar) buffer base, each lane's row and chunk a 32-bit byte offset
    // (< 256 rows x ld x 2 bytes), the k-tile a scalar offset.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.A + (int64_t)m0 * p.lda), 0, 0x7FFFFFFF, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        Q8 ? static_cast<void*>(const_cast<uint8_t*>(reinterpret_cast<const uint8_t*>(p.B) + (int64_t)n0 * p.ldb))
           : static_cast<void*>(const_cast<uint16_t*>(p.B + (int64_t)n0 * p.ldb)),
        0, 0x7FFFFFFF, 0x00020000);
    uint32_t oa[8], ob[8];  // the first A_DMA / B_DMA used (a fixed size: captured by the lambdas below)
    // Q8: thread t stages codes [16 (t % 4), +16) of B rows t / 4 + 16 NW j
    // (j < 16 / NW) and their block scales; they are converted to bf16 and
    // written to the stage one k-tile later (qwrite).
    constexpr int QJ = 16 / NW, QROWS = 16 * NW;  // weight rows per thread; rows per pass
    const int qr = tid >> 2, qc = tid & 3;
    uint32_t oq[QJ];
    const float* qs[QJ];
#pragma unroll
    for (int j = 0; j < QJ; ++j) {
        const int n = min(n0 + qr + QROWS * j, p.N - 1);
        oq[j] = Q8 ? (uint32_t)((int64_t)(n - n0) * p.ldb + 16 * qc) : 0u;
        qs[j] = Q8 ? p.Bs + n + (int64_t)(qc >> 1) * p.ldbs : nullptr;
    }
    uint4 qcode[QJ];
    float qscale[QJ];
#pragma unroll
    for (int j = 0; j < A_DMA; ++j) {
        const int row = (BM / NW) * wave + 8 * j + (lane >> 3);
        const int c = (lane & 7) ^ swz8(row);
        oa[j] = (uint32_t)(((int64_t)(min(m0 + row, p.M - 1) - m0) * p.lda + c * 8) * 2);
    }
#pragma unroll
    for (int j = 0; j < B_DMA; ++j) {
        const int row = (256 / NW) * wave + 8 * j + (lane >> 3);
        const int c = (lane & 7) ^ swz8(row);
        ob[j] = (uint32_t)(((int64_t)(min(n0 + row, p.N - 1) - n0) * p.ldb + c * 8) * 2);
    }
    typedef __attribute__((address_space(3))) void* lds_ptr_t;
    auto qload = [&](int kt) {
#pragma unroll
        for (int j = 0; j < QJ; ++j) {
            const auto v = __builtin_amdgcn_raw_buffer_load_b128(rb, oq[j], kt * EBK, 0);
            qcode[j] = make_uint4(v[0], v[1], v[2], v[3]);
            qscale[j] = qs[j][(int64_t)(2 * kt) * p.ldbs];
        }
    };
    // B rows of k-tile (codes in qcode) as bf16 into stage s: chunk c of row
    // r at c ^ swz8(r), w = fma(u, d, -128 d) rounded to bf16 (dt_dequant's).
    auto qwrite = [&](int s) {
        uint8_t* bbase = smem + s * STAGEB + AOPB;
#pragma unroll
        for (int j = 0; j < QJ; ++j) {
            const int r = qr + QROWS * j;
            const float d = qscale[j], m = -128.0f * d;
            const uint32_t w4[4] = {qcode[j].x, qcode[j].y, qcode[j].z, qcode[j].w};
            uint32_t pk[8];
#pragma unroll
            for (int h = 0; h < 4; ++h) {
                float w[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) w[e] = __builtin_fmaf((float)((w4[h] >> (8 * e)) & 0xFFu), d, m);
                pk[2 * h] = pack_bf16x2(w[0], w[1]);
                pk[2 * h + 1] = pack_bf16x2(w[2], w[3]);
            }
            const int sw = swz8(r);
            *reinterpret_cast<uint4*>(bbase + r * EROWB + (((2 * qc) ^ sw) << 4)) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
            *reinterpret_cast<uint4*>(bbase + r * EROWB + (((2 * qc + 1) ^ sw) << 4)) =
                make_uint4(pk[4], pk[5], pk[6], pk[7]);
        }
    };
    auto issue = [&](int kt, int s) {
        uint8_t* abase = smem + s * STAGEB + (BM / NW) * wave * EROWB;
        uint8_t* bbase = smem + s * STAGEB + AOPB + (256 / NW) * wave * EROWB;
        const int koff = kt * EBK * 2;
        if constexpr (Q8) qload(kt);  // before the A DMA: waiting for the codes leaves the DMA in flight
#pragma unroll
        for (int j = 0; j < 8; ++j) {  // A and B rows alternately
            if (j < A_DMA)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(abase + 8 * j * EROWB), 16, oa[j], koff, 0,
                                                         0);
            if (!Q8 && j < B_DMA)
                __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(bbase + 8 * j * EROWB), 16, ob[j], koff, 0,
                                                         0);
        }
    };
    f32x16_t acc[FN][FM];
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.f;

    const int lrow = lane & 31, g = lane >> 5;
    // Per-fragment swizzle of the rows this lane reads (rows wn + 32 j + lrow
    // and wm + 32 i + lrow).
    int sb[FN], sa[FM];
#pragma unroll
    for (int j = 0; j < FN; ++j) sb[j] = swz8(wn + 32 * j + lrow);
#pragma unroll
    for (int i = 0; i < FM; ++i) sa[i] = swz8(wm + 32 * i + lrow);
    bf16x8_t wa[FN], xa[FM], wb[FN], xb[FM];
    auto read_ops = [&](int s, int kk, bf16x8_t (&wf)[FN], bf16x8_t (&xf)[FM]) {
        const uint8_t* As = smem + s * STAGEB;
        const uint8_t* Bs = As + AOPB;
        const int c = 2 * kk + g;
#pragma unroll
        for (int j = 0; j < FN; ++j)
            wf[j] = *reinterpret_cast<const bf16x8_t*>(Bs + (wn + 32 * j + lrow) * EROWB + ((c ^ sb[j]) << 4));
#pragma unroll
        for (int i = 0; i < FM; ++i)
            xf[i] = *reinterpret_cast<const bf16x8_t*>(As + (wm + 32 * i + lrow) * EROWB + ((c ^ sa[i]) << 4));
    };
    auto mfma = [&](const bf16x8_t (&wf)[FN], const bf16x8_t (&xf)[FM]) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < FM; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j], xf[i], acc[j][i], 0, 0, 0);
    };
    // After read_ops(next) + mfma(current): {1 LDS read, 1 MFMA} per operand,
    // then the remaining MFMAs, so the last read has several MFMAs to land in.
    auto pipe = [&]() {
        if constexpr (SCHED) {
#pragma unroll
            for (int r = 0; r < FN + FM; ++r) {
                __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);  // DS read
                __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            }
            __builtin_amdgcn_sched_group_barrier(0x008, FN * FM - (FN + FM), 0);
        }
    };

    const int nk = p.K / EBK;
    issue(0, 0);
    if constexpr (Q8) qwrite(0);
    if (nk > 1) issue(1, 1);
    if (nk > 1) wait_vm<A_DMA + B_DMA>();  // Q8: QJ code and QJ scale loads stand in for the B_DMA B DMAs
    else wait_vm<0>();
    if constexpr (Q8) __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): the B rows written
    __builtin_amdgcn_s_barrier();
    read_ops(0, 0, wa, xa);
    // One k-tile: its four k-steps, each step's MFMAs running while the next
    // step's operands are read.  ISSUE: stage s is refilled with k-tile kt + 2
    // after the barrier (the last two k-tiles issue nothing); the peeled last
    // k-tile has no barrier.  Kept branch-free inside, so the DMA
    // instructions interleave with the step-3 MFMAs.
    auto body = [&](int kt, auto issue_next) {
        const int s = kt & 1;
        read_ops(s, 1, wb, xb);
        mfma(wa, xa);
        pipe();
        read_ops(s, 2, wa, xa);
        mfma(wb, xb);
        pipe();
        read_ops(s, 3, wb, xb);
        if constexpr (Q8) qwrite(s ^ 1);  // k-tile kt + 1's weights
        mfma(wa, xa);
        pipe();
        // Stage s is refilled with k-tile kt + 2 once every wave's reads of
        // it have returned; k-tile kt + 1 (the other stage) must have landed.
        wait_vm<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        if constexpr (decltype(issue_next)::value) issue(kt + 2, s);
        read_ops(s ^ 1, 0, wa, xa);
        mfma(wb, xb);
        if constexpr (SCHED) {
            // the DMA instructions one per MFMA, then the next step's reads
            constexpr int NDMA = decltype(issue_next)::value ? A_DMA + B_DMA : 0;
#pragma unroll
            for (int r = 0; r < (NDMA > FN * FM ? NDMA : FN * FM); ++r) {
                if (r < NDMA) __builtin_amdgcn_sched_group_barrier(0x020, 1, 0);    // VMEM read (DMA)
                if (r < FN * FM) __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // MFMA
            }
        }
    };
    for (int kt = 0; kt < nk - 2; ++kt) body(kt, std::true_type{});
    if (nk >= 2) body(nk - 2, std::false_type{});
    {
        const int s = (nk - 1) & 1;
        read_ops(s, 1, wb, xb);
        mfma(wa, xa);
        pipe();
        read_ops(s, 2, wa, xa);
        mfma(wb, xb);
        pipe();
        read_ops(s, 3, wb, xb);
        mfma(wa, xa);
        pipe();
        mfma(wb, xb);
    }
    epilogue<FM, FN, TC>(p, acc, m0 + wm, n0 + wn, lane);
}

// ---- Q8_0 weights: 256 x 256, 8 waves of 128 x 64, K = 64, 3 stages -----------
// The weight operand stays Q8_0 in HBM, in the split layout of
// dt_q8_0_split: uint8 codes u = q + 128 ([N][K], 1 byte per weight) and the
// fp32 block scales transposed ([K/32][N]).  A stage holds 256 A rows x 128 B
// (bf16, swizzled as in gemm_k64_kernel), 256 B rows x 64 B (codes) and the
// 2 x 256 scales of its two k-blocks: 50 KB, so three stages fit in LDS.
// Each B fragment is dequantised in registers, w = fma(u, d, -128 d) = d * q
// (exact in fp32: 11-bit x 8-bit significands), then rounded to bf16 by
// v_cvt_pk_bf16_f32 -- the same bf16 weights dt_dequant writes -- and fed to
// the same MFMA sequence as gemm_k64_kernel, so the result equals dt_dequant
// followed by the bf16 GEMM bit for bit.
// Eight waves, two per SIMD: each code is converted by the two waves that
// share its weight rows, but one wave's conversion (VALU) overlaps the other
// wave's MFMAs.  Measured on gfx950 at 4608 x {3072, 27648} x 3072: 90-93% of
// the bf16 GEMM's rate, against 70-78% for four waves of 256 x 64 (one per
// SIMD, each code converted once) with the conversion serialised behind the
// wave's own MFMAs, with or without explicit MFMA/VALU interleaving.
// B rows of 64 bytes: chunk kk of row n at kk ^ ((n >> 2) & 3), which makes
// the 16-byte reads of 16 consecutive rows at one chunk hit distinct banks.
constexpr int QBK = 64, QA_ROWB = QBK * 2, QA_OPB = 256 * QA_ROWB;  // 32 KB
constexpr int QB_ROWB = QBK, QB_OPB = 256 * QB_ROWB;               // 16 KB
constexpr int QS_OPB = 2 * 256 * 4;                                 // 2 KB
constexpr int QSTAGEB = QA_OPB + QB_OPB + QS_OPB, QSTAGES = 3;
constexpr int QDMA = 4 + 2 + 1;  // DMA instructions per wave per stage: A, B, scales

__device__ __forceinline__ int qswz(int n) { return (n >> 2) & 3; }

template <typename TC>
__global__ __launch_bounds__(512) void gemm_q8_kernel(const Group grp) {
    constexpr int FM = 4, FN = 2;  // wave sub-tile 128 (m) x 64 (n)
    __shared__ __attribute__((aligned(16))) uint8_t smem[QSTAGES * QSTAGEB];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar LDS destinations
    int tm, tn;
    const Problem& p = locate<256, 256>(grp, &tm, &tn);
    const int m0 = tm * 256, n0 = tn * 256;
    const int wm = (wave >> 2) * 128, wn = (wave & 3) * 64;

    // DMA sources.  A: wave w fills rows [32 w, +32), 4 instructions of 8 rows
    // (lane i: row + i / 8, chunk i % 8).  B: the same rows, 2 instructions of
    // 16 rows (lane i: row + i / 4, chunk i % 4).  Scales: the 64 scales of
    // k-block w / 4 for rows 64 (w % 4) + i, 4 bytes a lane, so every wave
    // issues the same QDMA instructions with every lane active.  Buffer loads
    // to LDS: the tile's first row (first scale) is the scalar buffer base,
    // each lane's part a 32-bit byte offset, the k-tile a scalar offset.
    const __amdgpu_buffer_rsrc_t ra = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.A + (int64_t)m0 * p.lda), 0, 0x7FFFFFFF, 0x00020000);
    const __amdgpu_buffer_rsrc_t rb = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint8_t*>(reinterpret_cast<const uint8_t*>(p.B) + (int64_t)n0 * p.ldb), 0, 0x7FFFFFFF,
        0x00020000);
    const __amdgpu_buffer_rsrc_t rs =
        __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(p.Bs), 0, 0x7FFFFFFF, 0x00020000);
    uint32_t oa[4], ob[2];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = 32 * wave + 8 * j + (lane >> 3);
        const int c = (lane & 7) ^ swz8(row);
        oa[j] = (uint32_t)(((int64_t)(min(m0 + row, p.M - 1) - m0) * p.lda + c * 8) * 2);
    }
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int row = 32 * wave + 16 * j + (lane >> 2);
        const int c = (lane & 3) ^ qswz(row);
        ob[j] = (uint32_t)((int64_t)(min(n0 + row, p.N - 1) - n0) * p.ldb + c * 16);
    }
    const int sblk = wave >> 2;
    const uint32_t os = (uint32_t)(((int64_t)sblk * p.ldbs + min(n0 + 64 * (wave & 3) + lane, p.N - 1)) * 4);
    const int s_lds = QA_OPB + QB_OPB + sblk * 1024 + 256 * (wave & 3);
    typedef __attribute__((address_space(3))) void* lds_ptr_t;
    auto issue = [&](int kt, int s) {
        uint8_t* st = smem + s * QSTAGEB;
        const int k0 = kt * QBK;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (lds_ptr_t)(st + (32 * wave + 8 * j) * QA_ROWB), 16, oa[j],
                                                     k0 * 2, 0, 0);
#pragma unroll
        for (int j = 0; j < 2; ++j)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (lds_ptr_t)(st + QA_OPB + (32 * wave + 16 * j) * QB_ROWB),
                                                     16, ob[j], k0, 0, 0);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_ptr_t)(st + s_lds), 4, os,
                                                 (int)((int64_t)(2 * kt) * p.ldbs * 4), 0, 0);
    };

    f32x16_t acc[FN][FM];
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.f;

    const int lrow = lane & 31, g = lane >> 5;
    int sa[FM], bofs[FN], qsw[FN];
#pragma unroll
    for (int i = 0; i < FM; ++i) sa[i] = swz8(wm + 32 * i + lrow);
#pragma unroll
    for (int j = 0; j < FN; ++j) {
        const int n = wn + 32 * j + lrow;
        bofs[j] = n * QB_ROWB;
        qsw[j] = qswz(n);
    }
    bf16x8_t wa[FN], xa[FM], wb[FN], xb[FM];
    uint2 braw[FN];
    float dsc[FN];
    // Operands of k-step kk (16 of K) of the k-tile in stage s: activations
    // straight from LDS, this lane's 8 weight codes and their scale into
    // registers.
    auto load_ops = [&](int s, int kk, bf16x8_t (&xf)[FM]) {
        const uint8_t* As = smem + s * QSTAGEB;
        const uint8_t* Bs_ = As + QA_OPB;
        const float* Ss = reinterpret_cast<const float*>(As + QA_OPB + QB_OPB) + (kk >> 1) * 256;
        const int c = 2 * kk + g;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            braw[j] = *reinterpret_cast<const uint2*>(Bs_ + bofs[j] + ((kk ^ qsw[j]) << 4) + 8 * g);
            dsc[j] = Ss[wn + 32 * j + lrow];
        }
#pragma unroll
        for (int i = 0; i < FM; ++i)
            xf[i] = *reinterpret_cast<const bf16x8_t*>(As + (wm + 32 * i + lrow) * QA_ROWB + ((c ^ sa[i]) << 4));
    };
    auto convert = [&](bf16x8_t (&wf)[FN]) {
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const uint32_t lo = braw[j].x, hi = braw[j].y;
            const float d = dsc[j], m = -128.0f * d;
            float w[8];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                w[e] = __builtin_fmaf((float)((lo >> (8 * e)) & 0xFFu), d, m);
                w[4 + e] = __builtin_fmaf((float)((hi >> (8 * e)) & 0xFFu), d, m);
            }
            wf[j] = __builtin_bit_cast(bf16x8_t, make_uint4(pack_bf16x2(w[0], w[1]), pack_bf16x2(w[2], w[3]),
                                                            pack_bf16x2(w[4], w[5]), pack_bf16x2(w[6], w[7])));
        }
    };
    auto mfma = [&](const bf16x8_t (&wf)[FN], const bf16x8_t (&xf)[FM]) {
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < FM; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j], xf[i], acc[j][i], 0, 0, 0);
    };

    const int nk = p.K / QBK;
#pragma unroll
    for (int s = 0; s < QSTAGES; ++s)
        if (s < nk) issue(s, s);
    // k-tile 0 landed, with min(nk - 1, 2) later k-tiles still in flight.
    if (nk >= 3) wait_vm<2 * QDMA>();
    else if (nk == 2) wait_vm<QDMA>();
    else wait_vm<0>();
    __builtin_amdgcn_s_barrier();
    load_ops(0, 0, xa);
    convert(wa);
    int st = 0;  // stage of k-tile kt
    // One k-tile: k-steps 0..3 of stage st (each reads the next k-step's
    // operands, runs this one's MFMAs and converts the next one's codes),
    // then the switch to the next stage.  `last`: k-tile kt + 1 is the final
    // one (nothing in flight after it, nothing more to issue).
    auto tile = [&](int kt, auto last) {
        load_ops(st, 1, xb);
        mfma(wa, xa);
        convert(wb);
        load_ops(st, 2, xa);
        mfma(wb, xb);
        convert(wa);
        load_ops(st, 3, xb);
        mfma(wa, xa);
        convert(wb);
        if constexpr (last.value) wait_vm<0>();
        else wait_vm<QDMA>();
        // Every wave's reads of stage st have returned before any wave passes
        // the barrier, so it can take k-tile kt + 3.
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        if constexpr (!last.value)
            if (kt + QSTAGES < nk) issue(kt + QSTAGES, st);
        st = st == QSTAGES - 1 ? 0 : st + 1;
        load_ops(st, 0, xa);
        mfma(wb, xb);
        convert(wa);
    };
    for (int kt = 0; kt < nk - 2; ++kt) tile(kt, std::false_type{});
    if (nk >= 2) tile(nk - 2, std::true_type{});
    load_ops(st, 1, xb);
    mfma(wa, xa);
    convert(wb);
    load_ops(st, 2, xa);
    mfma(wb, xb);
    convert(wa);
    load_ops(st, 3, xb);
    mfma(wa, xa);
    convert(wb);
    mfma(wb, xb);
    epilogue<FM, FN, TC>(p, acc, m0 + wm, n0 + wn, lane);
}

// ---- 128 x 128, register-staged, 2 stages --------------------------------------
// Q8: the weight operand in the split layout (uint8 codes u = q + 128 and fp32
// block scales), dequantised as it is staged: each thread converts 16 codes of
// one row, w = fma(u, d, -128 d) = d * q (exact) rounded to bf16 -- the value
// dt_dequant writes -- so LDS holds the bf16 operand and the MFMA sequence is
// the bf16 kernel's.  Products with few 256 x 256 tiles (the 512 text tokens)
// keep four times as many workgroups as gemm_q8_kernel.
constexpr int SBK = 64;
constexpr int SLDSW = SBK + 8;  // padded LDS row, in bf16 elements

template <typename TC, bool Q8 = false>
__global__ __launch_bounds__(256) void gemm_128_kernel(const Group grp) {
    constexpr int FM = 2, FN = 2, T = 256;
    constexpr int CH = 128 * (SBK / 8) / T;  // 16-byte chunks per thread per operand
    constexpr int STAGE = 256 * SLDSW;
    __shared__ __attribute__((aligned(16))) uint16_t smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tm, tn;
    const Problem& p = locate<128, 128>(grp, &tm, &tn);
    const int m0 = tm * 128, n0 = tn * 128;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;

    const uint16_t* Ap = p.A;
    const uint16_t* Bp = p.B;
    const int64_t lda = p.lda, ldb = p.ldb;
    const int Mx = p.M - 1, Nx = p.N - 1;
    // Thread chunk r covers row (tid + T r) / 8, k-chunk tid % 8 of each operand.
    const int kc = tid & 7, row0 = tid >> 3;
    const uint16_t* ga = Ap + (int64_t)min(m0 + row0, Mx) * lda + kc * 8;
    const uint16_t* gb = Bp + (int64_t)min(n0 + row0, Nx) * ldb + kc * 8;
    int64_t oa[CH], ob[CH];  // row offsets relative to ga / gb
#pragma unroll
    for (int r = 0; r < CH; ++r) {
        oa[r] = ((int64_t)min(m0 + row0 + (T / 8) * r, Mx) - min(m0 + row0, Mx)) * lda;
        ob[r] = ((int64_t)min(n0 + row0 + (T / 8) * r, Nx) - min(n0 + row0, Nx)) * ldb;
    }
    uint4 ra0, ra1, ra2, ra3, rb0, rb1, rb2, rb3;
    static_assert(CH == 4, "four chunks per thread per operand");
    // Q8: thread t stages codes [16 (t % 4), +16) of weight rows t / 4 and
    // t / 4 + 64, with their block scales.
    const int qr = tid >> 2, qc = tid & 3;
    const uint8_t* gq = reinterpret_cast<const uint8_t*>(Bp) + (int64_t)min(n0 + qr, Nx) * ldb + 16 * qc;
    const int64_t oq = ((int64_t)min(n0 + qr + 64, Nx) - min(n0 + qr, Nx)) * ldb;
    const float* gs = Q8 ? p.Bs + min(n0 + qr, Nx) : nullptr;
    const int64_t os = (int64_t)min(n0 + qr + 64, Nx) - min(n0 + qr, Nx);
    float sq0 = 0.f, sq1 = 0.f;
    auto fetch = [&](int k0) {
        ra0 = *reinterpret_cast<const uint4*>(ga + oa[0] + k0);
        ra1 = *reinterpret_cast<const uint4*>(ga + oa[1] + k0);
        ra2 = *reinterpret_cast<const uint4*>(ga + oa[2] + k0);
        ra3 = *reinterpret_cast<const uint4*>(ga + oa[3] + k0);
        if constexpr (Q8) {
            rb0 = *reinterpret_cast<const uint4*>(gq + k0);
            rb1 = *reinterpret_cast<const uint4*>(gq + oq + k0);
            const int64_t blk = (k0 + 16 * qc) >> 5;
            sq0 = gs[blk * p.ldbs];
            sq1 = gs[blk * p.ldbs + os];
        } else {
            rb0 = *reinterpret_cast<const uint4*>(gb + ob[0] + k0);
            rb1 = *reinterpret_cast<const uint4*>(gb + ob[1] + k0);
            rb2 = *reinterpret_cast<const uint4*>(gb + ob[2] + k0);
            rb3 = *reinterpret_cast<const uint4*>(gb + ob[3] + k0);
        }
    };
    // 16 codes -> 16 bf16 weights (two 16-byte chunks)
    auto dq16 = [&](const uint4& u, float d, uint16_t* dst) {
        const float m = -128.0f * d;
        const uint32_t w4[4] = {u.x, u.y, u.z, u.w};
        uint32_t pk[8];
#pragma unroll
        for (int h = 0; h < 4; ++h) {
            float w[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) w[e] = __builtin_fmaf((float)((w4[h] >> (8 * e)) & 0xFFu), d, m);
            pk[2 * h] = pack_bf16x2(w[0], w[1]);
            pk[2 * h + 1] = pack_bf16x2(w[2], w[3]);
        }
        *reinterpret_cast<uint4*>(dst) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        *reinterpret_cast<uint4*>(dst + 8) = make_uint4(pk[4], pk[5], pk[6], pk[7]);
    };
    auto stash = [&](int s) {
        uint16_t* As = smem + s * STAGE + row0 * SLDSW + kc * 8;
        uint16_t* Bs = As + 128 * SLDSW;
        constexpr int RS = (T / 8) * SLDSW;  // LDS offset between a thread's chunks
        *reinterpret_cast<uint4*>(As) = ra0;
        *reinterpret_cast<uint4*>(As + RS) = ra1;
        *reinterpret_cast<uint4*>(As + 2 * RS) = ra2;
        *reinterpret_cast<uint4*>(As + 3 * RS) = ra3;
        if constexpr (Q8) {
            uint16_t* Bq = smem + s * STAGE + 128 * SLDSW + qr * SLDSW + 16 * qc;
            dq16(rb0, sq0, Bq);
            dq16(rb1, sq1, Bq + 64 * SLDSW);
        } else {
            *reinterpret_cast<uint4*>(Bs) = rb0;
            *reinterpret_cast<uint4*>(Bs + RS) = rb1;
            *reinterpret_cast<uint4*>(Bs + 2 * RS) = rb2;
            *reinterpret_cast<uint4*>(Bs + 3 * RS) = rb3;
        }
    };

    f32x16_t acc[FN][FM];
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.f;

    const int lrow = lane & 31, lk = (lane >> 5) * 8;
    const int nk = p.K / SBK;
    fetch(0);
    stash(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int s = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) fetch((kt + 1) * SBK);
        const uint16_t* As = smem + s * STAGE;
        const uint16_t* Bs = As + 128 * SLDSW;
#pragma unroll
        for (int kk = 0; kk < SBK; kk += 16) {
            bf16x8_t wf[FN], xf[FM];
#pragma unroll
            for (int j = 0; j < FN; ++j)
                wf[j] = *reinterpret_cast<const bf16x8_t*>(&Bs[(wn + 32 * j + lrow) * SLDSW + kk + lk]);
#pragma unroll
            for (int i = 0; i < FM; ++i)
                xf[i] = *reinterpret_cast<const bf16x8_t*>(&As[(wm + 32 * i + lrow) * SLDSW + kk + lk]);
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int i = 0; i < FM; ++i)
                    acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j], xf[i], acc[j][i], 0, 0, 0);
        }
        if (more) stash(s ^ 1);
        __syncthreads();
    }
    epilogue<FM, FN, TC>(p, acc, m0 + wm, n0 + wn, lane);
}

// ---- any shape: 128 x 128, K in steps of 16 under a bounds mask ---------------
// For the GEMMs the kernels above do not take: K not a multiple of 64 (ggml's
// mul_mat takes any K, e.g. a ResnetBlock2D's time-embedding projection with
// 16 inputs), leading dimensions or bases without 16-byte alignment, and Q8_0
// weights with K % 64 == 32.  Each thread loads 8 consecutive k of one A row
// and one B row element by element, with zeros past K, through one LDS stage;
// a Q8_0 weight element is d * (u - 128) (exact in fp32) rounded to bf16, the
// value dt_dequant writes.  Four waves of 64 x 64 on the same MFMA as the
// kernels above.  These shapes are small (they occur outside the step's
// projections), so the kernel is written for coverage, not rate.
template <typename TC, bool Q8>
__global__ __launch_bounds__(256) void gemm_any_kernel(const Group grp) {
    constexpr int FM = 2, FN = 2, LDW = 24;  // LDS row: 16 bf16 + 8 of padding (48 bytes)
    __shared__ __attribute__((aligned(16))) uint16_t sa[128 * LDW];
    __shared__ __attribute__((aligned(16))) uint16_t sb[128 * LDW];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tm, tn;
    const Problem& p = locate<128, 128>(grp, &tm, &tn);
    const int m0 = tm * 128, n0 = tn * 128;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const int row = tid >> 1, kh = (tid & 1) * 8;
    const int64_t am = min(m0 + row, p.M - 1), bn = min(n0 + row, p.N - 1);
    const uint16_t* arow = p.A + am * p.lda;
    const uint16_t* brow = p.B + bn * p.ldb;
    const uint8_t* qrow = reinterpret_cast<const uint8_t*>(p.B) + bn * p.ldb;

    f32x16_t acc[FN][FM];
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[j][i][e] = 0.f;

    const int lrow = lane & 31, lk = (lane >> 5) * 8;
    for (int k0 = 0; k0 < p.K; k0 += 16) {
        uint32_t av[4], bv[4];
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            uint32_t a2 = 0, b2 = 0;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const int k = k0 + kh + e + h;
                if (k < p.K) {
                    a2 |= (uint32_t)arow[k] << (16 * h);
                    uint32_t bb;
                    if constexpr (Q8) {
                        const float d = p.Bs[(int64_t)(k >> 5) * p.ldbs + bn];
                        bb = f32_to_bf16_bits(mul_rn(d, (float)((int)qrow[k] - 128)));
                    } else {
                        bb = brow[k];
                    }
                    b2 |= bb << (16 * h);
                }
            }
            av[e / 2] = a2;
            bv[e / 2] = b2;
        }
        __syncthreads();  // every wave's reads of the previous k-step are done
        *reinterpret_cast<uint4*>(&sa[row * LDW + kh]) = make_uint4(av[0], av[1], av[2], av[3]);
        *reinterpret_cast<uint4*>(&sb[row * LDW + kh]) = make_uint4(bv[0], bv[1], bv[2], bv[3]);
        __syncthreads();
        bf16x8_t wf[FN], xf[FM];
#pragma unroll
        for (int j = 0; j < FN; ++j)
            wf[j] = *reinterpret_cast<const bf16x8_t*>(&sb[(wn + 32 * j + lrow) * LDW + lk]);
#pragma unroll
        for (int i = 0; i < FM; ++i)
            xf[i] = *reinterpret_cast<const bf16x8_t*>(&sa[(wm + 32 * i + lrow) * LDW + lk]);
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
            for (int i = 0; i < FM; ++i)
                acc[j][i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(wf[j], xf[i], acc[j][i], 0, 0, 0);
    }
    epilogue<FM, FN, TC>(p, acc, m0 + wm, n0 + wn, lane);
}

// ---- launch ---------------------------------------------------------------------

struct Config {
    int bm, bn, threads, per_cu;
    double rate;  // measured per-CU rate when the CUs are full (PFLOP/s, gfx950)
};
// 0: 256 x 256, 8 waves, K = 32 stages (one workgroup per CU); 1: 128 x 128
// (two per CU); 2: 256 x 256, 4 waves, K = 64 stages; 3: Q8_0 weights,
// 256 x 256, 8 waves, K = 64, three stages; 4: any shape (masked, 128 x 128);
// 5: config 2 with the operand reads interleaved into the MFMA stream; 6: the
// same at 224 x 256; 7: config 5 with Q8_0 weights dequantised as they are
// staged; 8, 9: configs 5 and 7 in eight waves of 128 x 64 (two per SIMD).
constexpr int kAnyConfig = 4, kLastConfig = 9;
constexpr Config kConfigs[10] = {{256, 256, 512, 1, 1.15}, {128, 128, 256, 2, 0.9}, {256, 256, 256, 1, 1.15},
                                {256, 256, 512, 1, 1.0},  {128, 128, 256, 2, 0.1}, {256, 256, 256, 1, 1.3},
                                {224, 256, 256, 1, 1.2},  {256, 256, 256, 1, 1.25}, {256, 256, 512, 1, 1.3},
                                {256, 256, 512, 1, 1.3}};

int64_t tiles_of(const Problem& p, int cfg) {
    const Config c = kConfigs[cfg];
    return (int64_t)((p.M + c.bm - 1) / c.bm) * ((p.N + c.bn - 1) / c.bn);
}

// Estimated time: ceil(tiles / concurrent workgroups) waves, each lasting the
// tile area x workgroups per CU / the per-CU rate, between the 256 x 256
// tiles (the scheduled K = 64 kernel, config 5: on gfx950 at M = 4608 it runs
// 1.01-1.14 PFLOP/s against 0.80-0.94 for the 8-wave kernel and 0.86-0.97
// for the unscheduled K = 64 kernel, bit-identical to the latter) and the
// 128 x 128 tiles.
// Whole-wave cost model: waves of tiles x tile area x workgroups per CU / rate.
int pick_by_waves(const Problem* ps, int n, int cus, std::initializer_list<int> cands) {
    int best = *cands.begin();
    double best_t = 1e300;
    for (int cfg : cands) {
        const Config c = kConfigs[cfg];
        int64_t tiles = 0;
        for (int i = 0; i < n; ++i) tiles += tiles_of(ps[i], cfg);
        const int64_t slots = (int64_t)cus * c.per_cu;
        const int64_t waves = (tiles + slots - 1) / slots;
        const double t = (double)waves * c.bm * c.bn * c.per_cu / c.rate;
        if (t < best_t) {
            best_t = t;
            best = cfg;
        }
    }
    return best;
}

// Q8_0 weights: the eight-wave K = 64 kernel's 256 x 256 tiles with the
// weights dequantised as they are staged (config 9) or, when those leave most
// CUs idle (the 512 text tokens' 3072-column products, a 128-column output),
// 128 x 128 tiles dequantised the same way (512 x 3072 x 9216: 135 against
// 203 us).
int pick_config_q8(const Problem* ps, int n, int cus) { return pick_by_waves(ps, n, cus, {9, 1}); }

// bf16 weights: the eight-wave K = 64 kernel's 256 x 256 tiles (config 8), or
// 128 x 128 tiles for the products with few tiles.  Config 8 measured faster
// than the four-wave 224 x 256 tiles on every product of the step that those
// took (4608 x 3072 x 9216: 210 against 225 us; 4608 x 3072 x 3072: 81.5
// against 91.6 us), so they are no longer a candidate.
int pick_config(const Problem* ps, int n, int cus) { return pick_by_waves(ps, n, cus, {8, 1}); }

template <typename TC>
int launch(const Problem* ps, int n, int cfg, hipStream_t st) {
    Group g{};
    g.count = n;
    int64_t total = 0;
    for (int i = 0; i < n; ++i) {
        g.p[i] = ps[i];
        g.tile_start[i] = (int)total;
        total += tiles_of(ps[i], cfg);
    }
    DT_REQUIRE(total < (1ll << 31), "dt_gemm_bf16: too many tiles");
    g.tile_start[n] = (int)total;
    if (total == 0) return DT_OK;
    const dim3 grid((unsigned)total), block((unsigned)kConfigs[cfg].threads);
    if (cfg == 0)
        hipLaunchKernelGGL((gemm_dma256_kernel<TC>), grid, block, 0, st, g);
    else if (cfg == 2)
        hipLaunchKernelGGL((gemm_k64_kernel<TC, false, 256>), grid, block, 0, st, g);
    else if (cfg == 5)
        hipLaunchKernelGGL((gemm_k64_kernel<TC, true, 256>), grid, block, 0, st, g);
    else if (cfg == 6)
        hipLaunchKernelGGL((gemm_k64_kernel<TC, true, 224>), grid, block, 0, st, g);
    else if (cfg == 7)
        hipLaunchKernelGGL((gemm_k64_kernel<TC, true, 256, true>), grid, block, 0, st, g);
    else if (cfg == 8)
        hipLaunchKernelGGL((gemm_k64_kernel<TC, true, 256, false, 8>), grid, block, 0, st, g);
    else if (cfg == 9)
        hipLaunchKernelGGL((gemm_k64_kernel<TC, true, 256, true, 8>), grid, block, 0, st, g);
    else if (cfg == 3)
        hipLaunchKernelGGL((gemm_q8_kernel<TC>), grid, block, 0, st, g);
    else if (cfg == kAnyConfig && ps[0].Bs)
        hipLaunchKernelGGL((gemm_any_kernel<TC, true>), grid, block, 0, st, g);
    else if (cfg == kAnyConfig)
        hipLaunchKernelGGL((gemm_any_kernel<TC, false>), grid, block, 0, st, g);
    else if (ps[0].Bs)
        hipLaunchKernelGGL((gemm_128_kernel<TC, true>), grid, block, 0, st, g);
    else
        hipLaunchKernelGGL((gemm_128_kernel<TC>), grid, block, 0, st, g);
    return check_launch("dt_gemm_bf16");
}

// Checks a problem and says whether the tiled kernels take it (K % 64 == 0,
// 16-byte aligned operand rows); any other valid shape runs gemm_any_kernel.
int validate(const dt_gemm_problem& q, int32_t c_type, Problem* out, bool* tiled) {
    DT_REQUIRE(q.M >= 0 && q.N >= 0 && q.K > 0, "dt_gemm_bf16: bad shape");
    DT_REQUIRE(q.M < (1ll << 31) && q.N < (1ll << 31) && q.K < (1ll << 31), "dt_gemm_bf16: shape too large");
    *tiled = true;
    if (q.M > 0 && q.N > 0) {  // an empty problem's leading dimensions are never used
        DT_REQUIRE(q.lda >= q.K && q.ldb >= q.K && q.ldc >= q.N,
                   "dt_gemm_bf16: leading dimensions must cover the rows");
        if (q.b_scale) {
            DT_REQUIRE(q.K % 32 == 0, "dt_gemm_q8_0: K (%lld) must be a multiple of 32 (Q8_0 blocks)",
                       (long long)q.K);
            DT_REQUIRE(q.ld_scale >= q.N && (reinterpret_cast<uintptr_t>(q.b_scale) & 3) == 0,
                       "dt_gemm_bf16: Q8_0 scales must be 4-byte aligned with ld_scale >= N");
        }
        DT_REQUIRE(!q.addend || q.ldd >= q.N, "dt_gemm_bf16: ldd < N");
        DT_REQUIRE(q.A && q.B && q.C, "dt_gemm_bf16: null pointer");
        DT_REQUIRE((reinterpret_cast<uintptr_t>(q.A) & 1) == 0 && (q.b_scale || (reinterpret_cast<uintptr_t>(q.B) & 1) == 0),
                   "dt_gemm_bf16: bf16 operands must be 2-byte aligned");
        const int es = c_type == DT_TYPE_F32 ? 4 : 2;
        DT_REQUIRE(q.N % 4 != 0 || ((reinterpret_cast<uintptr_t>(q.C) % (4 * es)) == 0 && q.ldc % 4 == 0),
                   "dt_gemm_bf16: C must be %d-byte aligned with ldc %% 4 == 0", 4 * es);
        // bf16 B: ldb in elements, % 8; Q8_0 codes: ldb in bytes, % 16.
        const int64_t ldb_align = q.b_scale ? 16 : 8;
        *tiled = q.K % 64 == 0 && q.lda % 8 == 0 && q.ldb % ldb_align == 0 && aligned16(q.A) && aligned16(q.B);
    }
    *out = Problem{(const uint16_t*)q.A, (const uint16_t*)q.B, q.C, q.addend, q.bias, q.lda, q.ldb,
                   q.ldc, q.ldd, (int)q.M, (int)q.N, (int)q.K, q.b_scale, q.ld_scale};
    return DT_OK;
}

}  // namespace
}  // namespace dit

extern "C" int dt_gemm_bf16_grouped(const dt_gemm_problem* problems, int32_t count, int32_t c_type,
                                    int32_t config, dt_stream_t stream) {
    using namespace dit;
    DT_REQUIRE(c_type == DT_TYPE_BF16 || c_type == DT_TYPE_F32, "dt_gemm_bf16: c_type %d unsupported", c_type);
    DT_REQUIRE(config >= -1 && config <= kLastConfig, "dt_gemm_bf16: config %d out of range", config);
    DT_REQUIRE(count >= 0 && count <= kMaxGroup, "dt_gemm_bf16_grouped: count %d outside 0..%d", count,
               kMaxGroup);
    DT_REQUIRE(problems || count == 0, "dt_gemm_bf16_grouped: null problem list");
    Problem ps[kMaxGroup];
    int n = 0, n_q8 = 0;
    bool all_tiled = true;
    for (int i = 0; i < count; ++i) {
        Problem p;
        bool tiled = true;
        int rc = validate(problems[i], c_type, &p, &tiled);
        if (rc) return rc;
        n_q8 += p.Bs != nullptr;
        if (p.M > 0 && p.N > 0) {
            ps[n++] = p;
            all_tiled &= tiled;
        }
    }
    DT_REQUIRE(n_q8 == 0 || n_q8 == count, "dt_gemm_bf16_grouped: a group mixes Q8_0 and bf16 weights");
    const bool q8_config = config == 3 || config == 7 || config == 9;  // configurations for Q8_0 weights only
    DT_REQUIRE(config == -1 || config == kAnyConfig || config == 1 || (n_q8 > 0) == q8_config,
               "dt_gemm_bf16: config %d does not take %s weights", config, n_q8 ? "Q8_0" : "bf16");
    DT_REQUIRE(config == -1 || config == kAnyConfig || all_tiled,
               "dt_gemm_bf16: config %d needs K %% 64 == 0 and 16-byte aligned rows", config);
    if (n == 0) return DT_OK;
    const int cfg = config >= 0      ? config
                    : !all_tiled     ? kAnyConfig
                    : n_q8           ? pick_config_q8(ps, n, cu_count())
                                     : pick_config(ps, n, cu_count());
    hipStream_t st = (hipStream_t)stream;
    return c_type == DT_TYPE_F32 ? launch<float>(ps, n, cfg, st) : launch<bf16>(ps, n, cfg, st);
}

extern "C" int dt_gemm_bf16_config(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                                   int64_t M, int64_t N, int64_t K, const float* bias, const void* addend,
                                   int64_t ldd, int32_t c_type, int32_t config, dt_stream_t stream) {
    const dt_gemm_problem p{A, lda, B, ldb, C, ldc, addend, ldd, bias, M, N, K};
    return dt_gemm_bf16_grouped(&p, 1, c_type, config, stream);
}

extern "C" int dt_gemm_q8_0(const void* A, int64_t lda, const void* codes, int64_t ld_codes, const float* scales,
                            int64_t ld_scales, void* C, int64_t ldc, int64_t M, int64_t N, int64_t K, const float* bias,
                            const void* addend, int64_t ldd, int32_t c_type, dt_stream_t stream) {
    dt_gemm_problem p{A, lda, codes, ld_codes, C, ldc, addend, ldd, bias, M, N, K, scales, ld_scales};
    DT_REQUIRE(scales != nullptr || M == 0 || N == 0, "dt_gemm_q8_0: null scales");
    return dt_gemm_bf16_grouped(&p, 1, c_type, -1, stream);
}

extern "C" int dt_gemm_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, void* C, int64_t ldc,
                            int64_t M, int64_t N, int64_t K, const float* bias, const void* addend,
                            int64_t ldd, int32_t c_type, dt_stream_t stream) {
    return dt_gemm_bf16_config(A, lda, B, ldb, C, ldc, M, N, K, bias, addend, ldd, c_type, -1, stream);
}
