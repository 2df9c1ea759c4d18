// gemm_f32.hip -- fp32 Linear and attention for graphs whose weights and
// activations are both F32, the reference's own precision (Linear::forward ->
// Runtime::mul_mat with F32 weights, src/nn/Linear.cpp:17-36; ggml computes
// such products in fp32), on the fp32 matrix cores of gfx950
// (v_mfma_f32_32x32x2_f32: products and sums in fp32).
//
// GEMM: C[m][n] = sum_k A[m][k] * B[n][k] (+ bias[n]) (+ D[m][n]), A the
// activation [M, K] and B the weight [N, K], both K-contiguous.  A workgroup
// of four waves computes a 128 x 128 tile, each wave 64 x 64 (2 x 2 blocks of
// 32 x 32), through K chunks of 16 staged in LDS (register-staged, double
// buffered).  As in the bf16 kernels the MFMA computes C^T = B A^T: the
// weight rows are the instruction's A operand, the activation rows its B
// operand, so lane l holds C[m = l % 32][n = 8 (i / 4) + 4 (l / 32) + i % 4]
// of each block and stores 4 consecutive n.  MFMA s of a chunk (s = 0..7)
// multiplies the k-pair {s, 8 + s}: lanes 0-31 supply k = s and lanes 32-63
// k = 8 + s, so each lane reads its 8 k of a row as two 16-byte LDS loads.
// The sum is blocked in two levels: MFMA s accumulates into set s % 2 of two
// running sets, and every 8 chunks (128 k) the two sets are added, (set 0 +
// set 1), into the tile's total and cleared.  A running set then adds at most
// 32 MFMA results of small partial sums and the total K/128 block sums, so
// fp32 rounding grows over about 32 + K/128 additions instead of K/2 for one
// chain (at K = 12288 one chain drifted 1.8e-5 from the fp64 sum, four sets
// of K/8 additions 1.0e-5), and the two sets' chains are independent, so an
// MFMA rarely waits on the previous one's result.
// Rows past M or N load a clamped valid row (products never stored); k past
// K loads zeros, so any K >= 1 is exact.
//
// Attention (no mask, head_dim 128): per (batch, head), S = Q K^T by the
// GEMM, P = softmax(scale S) row by row in fp32 (max, then expf(scale s - max),
// then the sum), O = P V by the GEMM against V^T (a transposed copy), heads
// taken eight at a time through a workspace -- the fp32 arithmetic of ggml's
// CPU flash_attn_ext for F32 operands (FlashAttentionOp.cpp:84-94), with the
// probabilities normalised before the product instead of after.
#include "capi_util.hpp"
#include "common.hpp"

namespace dit {
namespace {

typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kF32MaxGroup = 8;
constexpr int FT = 128;          // tile edge
constexpr int FKC = 16;          // K per chunk
constexpr int FKP = FKC + 4;     // padded LDS row, floats (80 bytes: 16 lanes' 16-byte reads hit distinct banks)

struct F32Problem {
    const float* A;
    const float* B;
    float* C;
    const float* D;
    const float* bias;
    int64_t lda, ldb, ldc, ldd;
    int M, N, K;
    int vec;  // 16-byte row loads allowed (K % 16 == 0, lda, ldb % 4 == 0, A and B 16-byte aligned)
};

struct F32Group {
    F32Problem p[kF32MaxGroup];
    int tile_start[kF32MaxGroup + 1];
    int count;
};

// This workgroup's problem and tile; XCD-contiguous numbering as in the bf16
// GEMM (each of the 8 XCDs takes a contiguous range of tiles).
__device__ __forceinline__ const F32Problem& f32_locate(const F32Group& g, int* tm, int* tn) {
    uint32_t bid = blockIdx.x;
    const uint32_t nb = gridDim.x, q = nb >> 3;
    if (bid < (q << 3)) bid = (bid & 7u) * q + (bid >> 3);
    int pi = 0;
    while (pi + 1 < g.count && (int)bid >= g.tile_start[pi + 1]) ++pi;
    const F32Problem& p = g.p[pi];
    const int local = (int)bid - g.tile_start[pi];
    const int tiles_n = (p.N + FT - 1) / FT;
    *tm = local / tiles_n;
    *tn = local - *tm * tiles_n;
    return p;
}

// 8 consecutive k of one row from k0, zeros past K.
__device__ __forceinline__ void load8(const float* row, int k0, int K, bool vec, float4& lo, float4& hi) {
    if (vec) {
        lo = *reinterpret_cast<const float4*>(row + k0);
        hi = *reinterpret_cast<const float4*>(row + k0 + 4);
        return;
    }
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = k0 + e < K ? row[k0 + e] : 0.0f;
    lo = make_float4(v[0], v[1], v[2], v[3]);
    hi = make_float4(v[4], v[5], v[6], v[7]);
}

__global__ __launch_bounds__(256) void gemm_f32_kernel(const F32Group grp) {
    constexpr int FM = 2, FN = 2;
    __shared__ __attribute__((aligned(16))) float sa[2][FT * FKP];
    __shared__ __attribute__((aligned(16))) float sb[2][FT * FKP];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    int tm, tn;
    const F32Problem& p = f32_locate(grp, &tm, &tn);
    const int m0 = tm * FT, n0 = tn * FT;
    const int wm = (wave >> 1) * 64, wn = (wave & 1) * 64;
    const bool vec = p.vec != 0;
    // Staging: thread t loads k [8 (t & 1), + 8) of row t >> 1 of both operands.
    const int row = tid >> 1, kh = (tid & 1) * 8;
    const float* arow = p.A + (int64_t)min(m0 + row, p.M - 1) * p.lda;
    const float* brow = p.B + (int64_t)min(n0 + row, p.N - 1) * p.ldb;

    constexpr int NSET = 2, FLUSH = 8;  // running sets; chunks per block sum
    f32x16_t acc[NSET][FN][FM], tot[FN][FM];
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int e = 0; e < 16; ++e) {
                tot[j][i][e] = 0.f;
#pragma unroll
                for (int c = 0; c < NSET; ++c) acc[c][j][i][e] = 0.f;
            }

    float4 ra0, ra1, rb0, rb1;
    auto fetch = [&](int k0) {
        load8(arow, k0 + kh, p.K, vec, ra0, ra1);
        load8(brow, k0 + kh, p.K, vec, rb0, rb1);
    };
    auto stash = [&](int s) {
        float* a = &sa[s][row * FKP + kh];
        float* b = &sb[s][row * FKP + kh];
        *reinterpret_cast<float4*>(a) = ra0;
        *reinterpret_cast<float4*>(a + 4) = ra1;
        *reinterpret_cast<float4*>(b) = rb0;
        *reinterpret_cast<float4*>(b + 4) = rb1;
    };

    const int lrow = lane & 31, lk = (lane >> 5) * 8;
    const int nk = (p.K + FKC - 1) / FKC;
    fetch(0);
    stash(0);
    __syncthreads();
    for (int kt = 0; kt < nk; ++kt) {
        const int s = kt & 1;
        const bool more = kt + 1 < nk;
        if (more) fetch((kt + 1) * FKC);
        float4 w[FN][2], x[FM][2];
#pragma unroll
        for (int j = 0; j < FN; ++j) {
            const float* r = &sb[s][(wn + 32 * j + lrow) * FKP + lk];
            w[j][0] = *reinterpret_cast<const float4*>(r);
            w[j][1] = *reinterpret_cast<const float4*>(r + 4);
        }
#pragma unroll
        for (int i = 0; i < FM; ++i) {
            const float* r = &sa[s][(wm + 32 * i + lrow) * FKP + lk];
            x[i][0] = *reinterpret_cast<const float4*>(r);
            x[i][1] = *reinterpret_cast<const float4*>(r + 4);
        }
#pragma unroll
        for (int st = 0; st < 8; ++st) {
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const float wv = w[j][st >> 2][st & 3];
#pragma unroll
                for (int i = 0; i < FM; ++i)
                    acc[st % NSET][j][i] =
                        __builtin_amdgcn_mfma_f32_32x32x2f32(wv, x[i][st >> 2][st & 3], acc[st % NSET][j][i], 0, 0, 0);
            }
        }
        if ((kt + 1) % FLUSH == 0 || !more) {
#pragma unroll
            for (int j = 0; j < FN; ++j)
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int e = 0; e < 16; ++e) {
                        tot[j][i][e] += acc[0][j][i][e] + acc[1][j][i][e];
                        acc[0][j][i][e] = 0.f;
                        acc[1][j][i][e] = 0.f;
                    }
        }
        if (more) stash(s ^ 1);
        __syncthreads();
    }

    // Epilogue: bias, addend, store 4 consecutive n per lane where they fit.
    const int g = lane >> 5;
    const bool v4 = (p.N % 4) == 0;
#pragma unroll
    for (int i = 0; i < FM; ++i) {
        const int m = m0 + wm + 32 * i + lrow;
        if (m >= p.M) continue;
#pragma unroll
        for (int j = 0; j < FN; ++j) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int n = n0 + wn + 32 * j + 8 * q + 4 * g;
                if (n >= p.N) continue;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * q + e;
                    v[e] = tot[j][i][r];
                    if (p.bias && n + e < p.N) v[e] += p.bias[n + e];
                    if (p.D && n + e < p.N) v[e] += p.D[(int64_t)m * p.ldd + n + e];
                }
                float* dst = p.C + (int64_t)m * p.ldc + n;
                if (v4 && n + 4 <= p.N) {
                    *reinterpret_cast<float4*>(dst) = make_float4(v[0], v[1], v[2], v[3]);
                } else {
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        if (n + e < p.N) dst[e] = v[e];
                }
            }
        }
    }
}

int64_t f32_tiles(const F32Problem& p) { return (int64_t)((p.M + FT - 1) / FT) * ((p.N + FT - 1) / FT); }

int f32_launch(const F32Problem* ps, int n, hipStream_t st) {
    F32Group g{};
    g.count = n;
    int64_t total = 0;
    for (int i = 0; i < n; ++i) {
        g.p[i] = ps[i];
        g.tile_start[i] = (int)total;
        total += f32_tiles(ps[i]);
    }
    DT_REQUIRE(total < (1ll << 31), "dt_gemm_f32: too many tiles");
    g.tile_start[n] = (int)total;
    if (total == 0) return DT_OK;
    hipLaunchKernelGGL(gemm_f32_kernel, dim3((unsigned)total), dim3(256), 0, st, g);
    return check_launch("dt_gemm_f32");
}

int f32_validate(const dt_gemm_problem& q, F32Problem* out) {
    DT_REQUIRE(q.M >= 0 && q.N >= 0 && q.K > 0, "dt_gemm_f32: bad shape");
    DT_REQUIRE(q.M < (1ll << 31) && q.N < (1ll << 31) && q.K < (1ll << 31), "dt_gemm_f32: shape too large");
    DT_REQUIRE(!q.b_scale, "dt_gemm_f32: F32 weights only");
    int vec = 0;
    if (q.M > 0 && q.N > 0) {
        DT_REQUIRE(q.lda >= q.K && q.ldb >= q.K && q.ldc >= q.N, "dt_gemm_f32: leading dimensions must cover the rows");
        DT_REQUIRE(!q.addend || q.ldd >= q.N, "dt_gemm_f32: ldd < N");
        DT_REQUIRE(q.A && q.B && q.C, "dt_gemm_f32: null pointer");
        DT_REQUIRE(((reinterpret_cast<uintptr_t>(q.A) | reinterpret_cast<uintptr_t>(q.B)) & 3) == 0,
                   "dt_gemm_f32: A and B must be 4-byte aligned");
        DT_REQUIRE(q.N % 4 != 0 || ((reinterpret_cast<uintptr_t>(q.C) & 15) == 0 && q.ldc % 4 == 0),
                   "dt_gemm_f32: C must be 16-byte aligned with ldc %% 4 == 0");
        vec = q.K % FKC == 0 && q.lda % 4 == 0 && q.ldb % 4 == 0 && aligned16(q.A) && aligned16(q.B);
    }
    *out = F32Problem{(const float*)q.A, (const float*)q.B, (float*)q.C, (const float*)q.addend, q.bias,
                      q.lda, q.ldb, q.ldc, q.ldd, (int)q.M, (int)q.N, (int)q.K, vec};
    return DT_OK;
}

// ---- attention pieces ---------------------------------------------------------

// dst[r][c] = src[c * src_ld + r] for a rows x cols block: V [Skv][128]
// (token stride src_ld) -> V^T [128][Skv]; 32 x 32 tiles through LDS.
__global__ __launch_bounds__(256) void transpose_f32_kernel(const float* __restrict__ src, int64_t src_ld,
                                                            float* __restrict__ dst, int rows, int cols) {
    __shared__ float t[32][33];
    const int c0 = blockIdx.x * 32, r0 = blockIdx.y * 32;
    const int tx = threadIdx.x & 31, ty = threadIdx.x >> 5;  // 32 x 8
    for (int k = ty; k < 32; k += 8) {
        const int c = c0 + k, r = r0 + tx;
        t[k][tx] = (c < cols && r < rows) ? src[(int64_t)c * src_ld + r] : 0.0f;
    }
    __syncthreads();
    for (int k = ty; k < 32; k += 8) {
        const int r = r0 + k, c = c0 + tx;
        if (r < rows && c < cols) dst[(int64_t)r * cols + c] = t[tx][k];
    }
}

// Row-wise softmax(scale * s) in place over rows of n: one workgroup per row.
__global__ __launch_bounds__(256) void softmax_rows_f32_kernel(float* __restrict__ s, int64_t n, float scale) {
    __shared__ float red[256 / kWave];
    float* row = s + (int64_t)blockIdx.x * n;
    float mx = -INFINITY;
    for (int64_t i = threadIdx.x; i < n; i += 256) mx = fmaxf(mx, scale * row[i]);
    // block max
    for (int off = 32; off > 0; off >>= 1) mx = fmaxf(mx, __shfl_xor(mx, off, kWave));
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    if (lane == 0) red[wid] = mx;
    __syncthreads();
    mx = red[0];
    for (int i = 1; i < 256 / kWave; ++i) mx = fmaxf(mx, red[i]);
    float sum = 0.0f;
    for (int64_t i = threadIdx.x; i < n; i += 256) {
        const float e = expf(scale * row[i] - mx);
        row[i] = e;
        sum += e;
    }
    sum = block_sum_f32(sum, red);
    const float inv = 1.0f / sum;
    for (int64_t i = threadIdx.x; i < n; i += 256) row[i] *= inv;
}

}  // namespace
}  // namespace dit

extern "C" int dt_gemm_f32_grouped(const dt_gemm_problem* problems, int32_t count, dt_stream_t stream) {
    using namespace dit;
    DT_REQUIRE(count >= 0 && count <= kF32MaxGroup, "dt_gemm_f32_grouped: count %d outside 0..%d", count,
               kF32MaxGroup);
    DT_REQUIRE(problems || count == 0, "dt_gemm_f32_grouped: null problem list");
    F32Problem ps[kF32MaxGroup];
    int n = 0;
    for (int i = 0; i < count; ++i) {
        F32Problem p;
        const int rc = f32_validate(problems[i], &p);
        if (rc) return rc;
        if (p.M > 0 && p.N > 0) ps[n++] = p;
    }
    if (n == 0) return DT_OK;
    return f32_launch(ps, n, (hipStream_t)stream);
}

extern "C" int dt_gemm_f32(const float* A, int64_t lda, const float* B, int64_t ldb, float* C, int64_t ldc, int64_t M,
                           int64_t N, int64_t K, const float* bias, const float* addend, int64_t ldd,
                           dt_stream_t stream) {
    const dt_gemm_problem p{A, lda, B, ldb, C, ldc, addend, ldd, bias, M, N, K, nullptr, 0};
    return dt_gemm_f32_grouped(&p, 1, stream);
}

// Workspace of dt_flash_attn_f32: per head of a group of up to 8, the
// scores [seq_q][seq_kv] and V^T [head_dim][seq_kv], fp32.
static int64_t attn_f32_group(int64_t batch, int64_t heads) {
    const int64_t bh = batch * heads;
    return bh < dit::kF32MaxGroup ? bh : dit::kF32MaxGroup;
}

extern "C" size_t dt_flash_attn_f32_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_q, int64_t seq_kv,
                                                     int64_t head_dim) {
    if (batch <= 0 || heads <= 0 || seq_q <= 0 || seq_kv <= 0 || head_dim <= 0) return 0;
    const int64_t per = (seq_q * seq_kv + head_dim * seq_kv + 3) / 4 * 4;  // 16-byte aligned per head
    return (size_t)(attn_f32_group(batch, heads) * per) * sizeof(float);
}

extern "C" int dt_flash_attn_f32(const float* q, const float* k, const float* v, float* o, int64_t batch,
                                 int64_t heads, int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                                 const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                                 const int64_t* o_strides, float scale, void* workspace, size_t workspace_bytes,
                                 dt_stream_t stream) {
    using namespace dit;
    DT_REQUIRE(batch >= 0 && heads >= 0 && seq_q >= 0 && seq_kv >= 0 && head_dim > 0,
               "dt_flash_attn_f32: bad shape");
    if (batch == 0 || heads == 0 || seq_q == 0) return DT_OK;
    DT_REQUIRE(seq_kv > 0, "dt_flash_attn_f32: no keys");
    DT_REQUIRE(q && k && v && o && q_strides && k_strides && v_strides && o_strides, "dt_flash_attn_f32: null pointer");
    DT_REQUIRE(seq_q < (1ll << 31) && seq_kv < (1ll << 31) && seq_q * seq_kv < (1ll << 40),
               "dt_flash_attn_f32: sequence too long");
    const size_t need = dt_flash_attn_f32_workspace_bytes(batch, heads, seq_q, seq_kv, head_dim);
    DT_REQUIRE(workspace && workspace_bytes >= need && aligned16(workspace),
               "dt_flash_attn_f32: workspace of %zu bytes (16-byte aligned) needed", need);
    hipStream_t st = (hipStream_t)stream;
    const int64_t per = (seq_q * seq_kv + head_dim * seq_kv + 3) / 4 * 4;
    const int64_t bh = batch * heads, gsz = attn_f32_group(batch, heads);
    float* ws = (float*)workspace;
    for (int64_t h0 = 0; h0 < bh; h0 += gsz) {
        const int n = (int)(bh - h0 < gsz ? bh - h0 : gsz);
        dt_gemm_problem sp[kF32MaxGroup], op[kF32MaxGroup];
        for (int i = 0; i < n; ++i) {
            const int64_t b = (h0 + i) / heads, h = (h0 + i) % heads;
            float* S = ws + i * per;
            float* Vt = S + seq_q * seq_kv;
            const float* qh = q + b * q_strides[0] + h * q_strides[2];
            const float* kh = k + b * k_strides[0] + h * k_strides[2];
            const float* vh = v + b * v_strides[0] + h * v_strides[2];
            float* oh = o + b * o_strides[0] + h * o_strides[2];
            // V^T [head_dim][seq_kv]
            const dim3 tg((unsigned)((seq_kv + 31) / 32), (unsigned)((head_dim + 31) / 32));
            hipLaunchKernelGGL(transpose_f32_kernel, tg, dim3(256), 0, st, vh, v_strides[1], Vt, (int)head_dim,
                               (int)seq_kv);
            int rc = check_launch("dt_flash_attn_f32(transpose)");
            if (rc) return rc;
            sp[i] = dt_gemm_problem{qh, q_strides[1], kh, k_strides[1], S, seq_kv, nullptr, 0, nullptr,
                                    seq_q, seq_kv, head_dim, nullptr, 0};
            op[i] = dt_gemm_problem{S, seq_kv, Vt, seq_kv, oh, o_strides[1], nullptr, 0, nullptr,
                                    seq_q, head_dim, seq_kv, nullptr, 0};
        }
        int rc = dt_gemm_f32_grouped(sp, n, stream);
        if (rc) return rc;
        for (int i = 0; i < n; ++i) {
            hipLaunchKernelGGL(softmax_rows_f32_kernel, dim3((unsigned)seq_q), dim3(256), 0, st, ws + i * per,
                               seq_kv, scale);
            rc = check_launch("dt_flash_attn_f32(softmax)");
            if (rc) return rc;
        }
        rc = dt_gemm_f32_grouped(op, n, stream);
        if (rc) return rc;
    }
    return DT_OK;
}
