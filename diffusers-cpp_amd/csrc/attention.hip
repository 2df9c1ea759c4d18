// attention.hip -- unmasked scaled-dot-product attention for head_dim 128,
// the op behind FlashAttentionOp::operator() (src/nn/attention/FlashAttentionOp.cpp:84-94,
// ggml_flash_attn_ext with scale 1/sqrt(128), no mask in Flux2):
//   O[s, :] = sum_j softmax_j(scale * <Q[s], K[j]>) V[j, :]   per (batch, head).
//
// Formulation (gfx950, v_mfma_f32_32x32x16_bf16): each wave owns 32 queries
// and computes the TRANSPOSED products S^T = K Q^T and O^T += V^T P^T, so the
// accumulator column -- the query -- is the lane index (lane % 32) in both.
// Every per-query softmax quantity (running max, running sum, rescale factor)
// is therefore a per-lane scalar, shared only with the partner lane l ^ 32
// that holds the other half of the keys.  P^T goes from the S^T accumulator
// registers straight into the B operand of the PV product: the MFMA's
// reduction index is a permutation of 16 keys, and V^T is read from LDS in
// that same permutation (keys {4g..4g+3, 8+4g..8+4g+3} for lane half g).
//
// A 256-thread workgroup (4 waves, 128 queries) shares 64-key K and V tiles
// in LDS, double-buffered and filled by direct DMA; two workgroups per CU
// give each SIMD two waves, so one wave's softmax overlaps the other's
// MFMAs.  Workgroups are ordered so that each XCD (8 per MI355X, one L2 each)
// works through a contiguous range of (batch, head) slices.
#include <math.h>

#include <algorithm>
#include <type_traits>

#include "capi_util.hpp"
#include "common.hpp"
#include "kernels.hpp"
#include "rope_angles.hpp"

namespace dit {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int D = 128;       // head dim
constexpr int QB = 128;      // queries per workgroup

struct AttnArgs {
    const uint16_t* q;
    const uint16_t* k;
    const uint16_t* v;
    void* o;
    int64_t qs[3], ks[3], vs[3], os[3];  // batch, token, head strides (elements)
    int32_t batch, heads, seq_q, seq_kv;
    int32_t q_blocks;                     // ceil(seq_q / QB)
    float scale_log2;                     // scale * log2(e)
};

// The Q prologue's operands: q before its QK-RMSNorm + RoPE, in up to two
// token segments with their own norm weights (the txt | img concatenation of
// Flux2Attention.hpp:93-116; one segment: split = seq_q), and the RoPE
// positions of the joint sequence.
struct AttnPro {
    const uint16_t* q0;
    const uint16_t* q1;
    int64_t q0_bs, q0_ts, q0_hs, q1_bs, q1_ts, q1_hs;  // batch, token, head strides (elements)
    const float* w0;
    const float* w1;
    int32_t split;       // queries [0, split) from q0, [split, seq_q) from q1 (token - split)
    int32_t axis_dim, n_pos;
    float theta_scale, eps;
    const float* table;  // [n_pos][axis_dim] (cos, sin); NULL: angles on the device
    RopeAxisPos pos;     // position of joint token t on axis a: pos.ptr[a][t * pos.stride[a]]
};

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// Position of token t on axis `axis`, through an unrolled select so the
// kernel-argument arrays are never indexed dynamically.
__device__ __forceinline__ int pro_position(const RopeAxisPos& pos, int axis, int t) {
    const int32_t* p = pos.ptr[0];
    int64_t st = pos.stride[0];
#pragma unroll
    for (int a = 1; a < kMaxRopeAxes; ++a)
        if (axis == a) {
            p = pos.ptr[a];
            st = pos.stride[a];
        }
    return p[(int64_t)t * st];
}

// Query `qrow` of the wave with QK-RMSNorm + RoPE applied, written as bf16
// to `row` (256 bytes of LDS): lane half g owns dims 16 c + 8 g + [0, 8) of
// chunk c, as in the B operand it is read back into.  Every operation is
// the QK kernel's (qk_rope.hip), in its order: per 8-dim chunk the sum of
// squares, the 16 chunk sums added as its 16-lane DPP tree does (pairs,
// quads, halves, whole), 1 / sqrt(ss / 128 + eps), (x * r) * w, the
// rotation, one bf16 rounding -- so the q used here is bit-identical to the
// stored output of dt_qk_rmsnorm_rope.  The chunk loop writes LDS rather than
// registers, so it need not unroll and adds nothing to the main loop's
// register budget; the second pass re-reads the chunks (cache hits).
__device__ __forceinline__ void q_prologue(const AttnPro& pro, int b, int h, int qrow, int seq_q, int g,
                                           uint8_t* row) {
    const bool valid = qrow < seq_q;
    const int seg = valid && qrow >= pro.split;
    const int tok = seg ? qrow - pro.split : qrow;
    const uint16_t* src = seg ? pro.q1 + b * pro.q1_bs + (int64_t)tok * pro.q1_ts + h * pro.q1_hs
                              : pro.q0 + b * pro.q0_bs + (int64_t)tok * pro.q0_ts + h * pro.q0_hs;
    // Every independent load first: the positions (their table rows are the
    // one dependent load), the 8 chunks of q.
    int p[8];
    bool hit = valid && pro.table != nullptr;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        const int d0 = 16 * c + 8 * g;
        p[c] = valid ? pro_position(pro.pos, d0 / pro.axis_dim, qrow) : 0;
    }
    uint4 raw[8];
    float part[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) raw[c] = valid ? ld16(src + 16 * c + 8 * g) : make_uint4(0, 0, 0, 0);
#pragma unroll
    for (int c = 0; c < 8; ++c) hit = hit && p[c] >= 0 && p[c] < pro.n_pos;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        float v[8];
        Io<bf16>::unpack(raw[c], v);
        float ss = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) ss += v[e] * v[e];
        part[c] = ss;
    }
    // Chunk 2 c + g is here, 2 c + (1 - g) in lane l ^ 32: their sum is the
    // tree's first level whichever half holds which.
    float s1[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) s1[c] = part[c] + __shfl_xor(part[c], 32);
    const float ss = ((s1[0] + s1[1]) + (s1[2] + s1[3])) + ((s1[4] + s1[5]) + (s1[6] + s1[7]));
    const float r = 1.0f / sqrtf(ss / (float)D + pro.eps);
    const float* w = seg ? pro.w1 : pro.w0;
    auto emit = [&](int c, const float* v, const float* cs) {
        const int d0 = 16 * c + 8 * g;
        float wv[8], o[8];
        const float4 wa = *reinterpret_cast<const float4*>(w + d0);
        const float4 wb = *reinterpret_cast<const float4*>(w + d0 + 4);
        wv[0] = wa.x; wv[1] = wa.y; wv[2] = wa.z; wv[3] = wa.w;
        wv[4] = wb.x; wv[5] = wb.y; wv[6] = wb.z; wv[7] = wb.w;
#pragma unroll
        for (int qd = 0; qd < 4; ++qd) {
            const float x0 = mul_rn(mul_rn(v[2 * qd], r), wv[2 * qd]);
            const float x1 = mul_rn(mul_rn(v[2 * qd + 1], r), wv[2 * qd + 1]);
            const float cn = cs[2 * qd], sn = cs[2 * qd + 1];
            o[2 * qd] = sub_rn(mul_rn(x0, cn), mul_rn(x1, sn));
            o[2 * qd + 1] = add_rn(mul_rn(x0, sn), mul_rn(x1, cn));
        }
        *reinterpret_cast<uint4*>(row + 2 * d0) = Io<bf16>::pack(o);
    };
    if (hit) {  // every angle from the table: unrolled, its loads issued together
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            const int d0 = 16 * c + 8 * g;
            const int i0 = d0 - (d0 / pro.axis_dim) * pro.axis_dim;
            const float* t = pro.table + (int64_t)p[c] * pro.axis_dim + i0;  // rope_angles' table branch
            const float4 ca = *reinterpret_cast<const float4*>(t), cb = *reinterpret_cast<const float4*>(t + 4);
            const float cs[8] = {ca.x, ca.y, ca.z, ca.w, cb.x, cb.y, cb.z, cb.w};
            float v[8];
            Io<bf16>::unpack(raw[c], v);
            emit(c, v, cs);
        }
    } else if (valid) {  // some angle off the table: the device recurrence
        for (int c = 0; c < 8; ++c) {
            const int d0 = 16 * c + 8 * g;
            const int axis = d0 / pro.axis_dim, i0 = d0 - axis * pro.axis_dim;
            float cs[8], v[8];
            rope_angles<4>(pro_position(pro.pos, axis, qrow), i0, pro.table, pro.n_pos, pro.axis_dim,
                           pro.theta_scale, cs);
            Io<bf16>::unpack(ld16(src + d0), v);
            emit(c, v, cs);
        }
    } else {
#pragma unroll
        for (int c = 0; c < 8; ++c) *reinterpret_cast<uint4*>(row + 2 * (16 * c + 8 * g)) = make_uint4(0, 0, 0, 0);
    }
}

// ---- K/V by direct DMA, two workgroups per CU ---------------------------------
// K and V tiles move global -> LDS by direct DMA (global_load_lds_dwordx4)
// into two 32 KB buffers, so no registers are spent on staging.  At most 256 registers per lane (two waves per SIMD):
// one wave's softmax (VALU) runs while the other wave on the SIMD issues
// MFMAs.  V stays [key][d] in LDS; the V^T A operand is read with
// ds_read_tr16_b64, which gives lane i of a 16-lane group element c = i % 4
// of lane 4 j + i / 4's 4 x b16: with lane s addressing V[k0 + s / 4][d0 +
// 4 (s % 4) ..], lane i receives V[k0 + j][d0 + i] for j = 0..3, i.e. four
// keys of one d.  Rows of 256 bytes are XOR-swizzled in 16-byte chunks:
// K chunk c of row r at c ^ (r & 15) (16 rows read one logical chunk),
// V chunk c at c ^ 4 (r & 3) (4 rows x 4 consecutive chunks per transposed
// read).
constexpr int DKB = 64;                 // keys per tile
constexpr int DROW = D * 2;             // bytes per K / V row
constexpr int DTILE = DKB * DROW;       // 16 KB

__device__ __forceinline__ int kswz(int r) { return r & 15; }
__device__ __forceinline__ int vswz(int r) { return (r & 3) << 2; }

template <int N_OUT>
__device__ __forceinline__ void attn_wait_vm() {
    __builtin_amdgcn_s_waitcnt((N_OUT & 15) | ((N_OUT >> 4) << 14) | 0x0F70);
}

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4_t* lds_short4_p;

// ds_read_tr16_b64 of the 8 bytes at p (an LDS address).
__device__ __forceinline__ uint2 read_tr16(const uint8_t* p) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4_p)(p)));
}

template <typename TO, bool PRO>
__global__ __launch_bounds__(256, 2) void flash_attn_dma_kernel(AttnArgs a, AttnPro pro) {
    // [buffer][K | V][64 rows][256 B]
    __shared__ __attribute__((aligned(16))) uint8_t smem[2 * 2 * DTILE];

    uint32_t bid = blockIdx.x;
    const uint32_t nb = gridDim.x;
    if ((nb & 7u) == 0) bid = (bid & 7u) * (nb >> 3) + (bid >> 3);
    const int qblk = (int)(bid % (uint32_t)a.q_blocks);
    const int bh = (int)(bid / (uint32_t)a.q_blocks);
    const int h = bh % a.heads, b = bh / a.heads;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 31, g = lane >> 5;
    const int q0 = qblk * QB + wave * 32;

    const uint16_t* Qp = a.q + b * a.qs[0] + h * a.qs[2];
    const uint16_t* Kp = a.k + b * a.ks[0] + h * a.ks[2];
    const uint16_t* Vp = a.v + b * a.vs[0] + h * a.vs[2];

    bf16x8_t qf[8];
    if constexpr (!PRO) {
        const int qrow = q0 + r;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            uint4 u = qrow < a.seq_q ? ld16(Qp + (int64_t)qrow * a.qs[1] + 16 * c + 8 * g) : make_uint4(0, 0, 0, 0);
            qf[c] = __builtin_bit_cast(bf16x8_t, u);
        }
    }

    // DMA: wave w fills rows [16 w, 16 w + 16) of the K and the V tile, four
    // instructions of 4 rows each; lane i covers row + i / 16, stored chunk
    // i % 16, loaded from the swizzled source chunk.  Rows past seq_kv load
    // the last valid row (finite data; their scores are masked).
    const int drow = 16 * wave + (lane >> 4), dpos = lane & 15;
    const uint16_t* kq[4];
    const uint16_t* vq[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int row = drow + 4 * j;
        kq[j] = Kp + (int64_t)row * a.ks[1] + (dpos ^ kswz(row)) * 8;
        vq[j] = Vp + (int64_t)row * a.vs[1] + (dpos ^ vswz(row)) * 8;
    }
    auto issue = [&](int kv0, int buf) {
        uint8_t* kb = smem + buf * 2 * DTILE + 16 * wave * DROW;
        uint8_t* vb = kb + DTILE;
        if (kv0 + DKB <= a.seq_kv) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                __builtin_amdgcn_global_load_lds(kq[j] + (int64_t)kv0 * a.ks[1], kb + 4 * j * DROW, 16, 0, 0);
                __builtin_amdgcn_global_load_lds(vq[j] + (int64_t)kv0 * a.vs[1], vb + 4 * j * DROW, 16, 0, 0);
            }
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int row = drow + 4 * j;
                const int key = min(kv0 + row, a.seq_kv - 1);
                __builtin_amdgcn_global_load_lds(Kp + (int64_t)key * a.ks[1] + (dpos ^ kswz(row)) * 8,
                                                 kb + 4 * j * DROW, 16, 0, 0);
                __builtin_amdgcn_global_load_lds(Vp + (int64_t)key * a.vs[1] + (dpos ^ vswz(row)) * 8,
                                                 vb + 4 * j * DROW, 16, 0, 0);
            }
        }
    };

    // Per-lane LDS offsets, the same for every tile.  K: row 32 hh + r, chunk
    // 2 c + g at (2 c + g) ^ (r & 15) (32 hh is an immediate).  V (transposed
    // reads): lane s of 16-lane group gi reads row 16 j + 4 tg + s / 4 (+ 8),
    // d = 32 tt + 16 dsub + 4 (s % 4), whose swizzled chunk is
    // 4 (tt ^ s / 4) + (16 dsub + 4 (s % 4)) / 8.
    int koff[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) koff[c] = r * DROW + (((2 * c + g) ^ (r & 15)) << 4);
    const int s16 = lane & 15, gi = lane >> 4, tg = gi >> 1, dsub = gi & 1;
    const int trow = s16 >> 2, tcol = 16 * dsub + 4 * (s16 & 3);
    int voff[4];
#pragma unroll
    for (int tt = 0; tt < 4; ++tt)
        voff[tt] = (4 * tg + trow) * DROW + ((4 * (tt ^ trow) + (tcol >> 3)) << 4) + 8 * ((tcol >> 2) & 1);

    f32x16_t o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[t][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;  // running max in units of scale * log2(e)
    const float sc = a.scale_log2;          // >= 0, so max(sc * s) = sc * max(s)

    const int ntiles = (a.seq_kv + DKB - 1) / DKB;
    auto tile = [&](int t, auto buf_c, auto mask_c) {
        constexpr int BUF = decltype(buf_c)::value;
        constexpr bool MASK = decltype(mask_c)::value;
        const int kv0 = t * DKB;
        // One barrier per tile: once every wave has this tile's DMA and has
        // finished the previous tile (its LDS reads returned), the previous
        // tile's buffer takes tile t + 1 while tile t is computed -- the same
        // slack as issuing it two tiles ahead after a second barrier at the
        // end of each tile, which measured 3% slower (271.7 -> 263.7 us at
        // 4608 x 4608 x 24 heads).
        attn_wait_vm<0>();
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
        __builtin_amdgcn_s_barrier();
        if (t + 1 < ntiles) issue(kv0 + DKB, BUF ^ 1);
        const uint8_t* Kt = smem + BUF * 2 * DTILE;
        const uint8_t* Vt_ = Kt + DTILE;

        // The two 32-key halves are independent accumulator chains; issuing
        // them alternately keeps the MFMA pipe from waiting on each result.
        f32x16_t sacc[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int e = 0; e < 16; ++e) sacc[hh][e] = 0.f;
#pragma unroll
        for (int c = 0; c < 8; ++c)
#pragma unroll
            for (int hh = 0; hh < 2; ++hh) {
                const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(Kt + 32 * hh * DROW + koff[c]);
                sacc[hh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[c], sacc[hh], 0, 0, 0);
            }
        // Element i of sacc[hh] is key kv0 + 32 hh + 8 (i / 4) + 4 g + i % 4.
        float mx = -INFINITY;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                if (MASK && kv0 + 32 * hh + 8 * (i >> 2) + 4 * g + (i & 3) >= a.seq_kv) continue;
                mx = fmaxf(mx, sacc[hh][i]);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        // The reference max moves only when a score exceeds it by more than
        // 2^8: every exponent argument stays <= 8, so P <= 256 (exact in bf16
        // range, no fp32 overflow), and O and l share the same reference, so
        // O / l is unchanged.  Most tiles then skip the 64 rescales.
        const float m_cand = fmaxf(m_run, mx * sc);
        const bool move = m_cand > m_run + 8.0f;
        if (__builtin_amdgcn_ballot_w64(move)) {
            const float m_new = move ? m_cand : m_run;
            const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
            l_run *= alpha;
#pragma unroll
            for (int tt = 0; tt < 4; ++tt)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[tt][e] *= alpha;
            m_run = m_new;
        }
        const float m_new = m_run;
        float psum = 0.f;
        bf16x8_t pf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int e = 0; e < 8; e += 2) {
                float p2[2];
#pragma unroll
                for (int u = 0; u < 2; ++u) {
                    const int i = 8 * (j & 1) + e + u;
                    float arg = __builtin_fmaf(sacc[j >> 1][i], sc, -m_new);
                    if (MASK && kv0 + 32 * (j >> 1) + 8 * (i >> 2) + 4 * g + (i & 3) >= a.seq_kv) arg = -INFINITY;
                    p2[u] = __builtin_amdgcn_exp2f(arg);
                    psum += p2[u];
                }
                const uint32_t pk = pack_bf16x2(p2[0], p2[1]);
                pf[j][e] = __builtin_bit_cast(__bf16, (uint16_t)(pk & 0xFFFFu));
                pf[j][e + 1] = __builtin_bit_cast(__bf16, (uint16_t)(pk >> 16));
            }
        }
        l_run += psum;

        // O^T[d][q] += V^T[d][key] P^T[key][q]: MFMA j covers keys 16 j ..;
        // lane half g supplies keys {16 j + 4 g + e, 16 j + 8 + 4 g + e}.
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int tt = 0; tt < 4; ++tt) {
                const uint2 lo = read_tr16(Vt_ + 16 * j * DROW + voff[tt]);
                const uint2 hi = read_tr16(Vt_ + (16 * j + 8) * DROW + voff[tt]);
                const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
                o[tt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[j], o[tt], 0, 0, 0);
            }
        }
    };

    using B0 = std::integral_constant<int, 0>;
    using B1 = std::integral_constant<int, 1>;
    using Full = std::integral_constant<bool, false>;
    using Part = std::integral_constant<bool, true>;
    // Full tiles in pairs (the buffer of each is then a constant), then the
    // last tile, masked when seq_kv is not a multiple of the tile.
    const int nfull = a.seq_kv / DKB;
    issue(0, 0);
    if constexpr (PRO) {
        // q goes through the second K/V buffer, still idle while the first
        // tile's DMA (above) is in flight: wave w's rows at [32 w, 32 w +
        // 32) x 256 B.  Every wave has read its rows back before the
        // barrier, and the buffer's first DMA comes after it.
        uint8_t* row = smem + 2 * DTILE + (32 * wave + r) * DROW;
        q_prologue(pro, b, h, q0 + r, a.seq_q, g, row);
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's rows are in LDS
#pragma unroll
        for (int c = 0; c < 8; ++c) qf[c] = *reinterpret_cast<const bf16x8_t*>(row + 2 * (16 * c + 8 * g));
        __syncthreads();
    }
    int t = 0;
    for (; t + 1 < nfull; t += 2) {
        tile(t, B0{}, Full{});
        tile(t + 1, B1{}, Full{});
    }
    if (t < nfull) {
        tile(t, B0{}, Full{});
        ++t;
        if (t < ntiles) tile(t, B1{}, Part{});
    } else if (t < ntiles) {
        tile(t, B0{}, Part{});
    }

    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = 1.0f / l_tot;
    const int q = q0 + r;
    if (q < a.seq_q) {
        TO* op = reinterpret_cast<TO*>(a.o) + b * a.os[0] + (int64_t)q * a.os[1] + h * a.os[2];
#pragma unroll
        for (int tt = 0; tt < 4; ++tt)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const int d = 32 * tt + 8 * i4 + 4 * g;
                float v4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = o[tt][4 * i4 + e] * inv;
                if constexpr (sizeof(TO) == 4) {
                    *reinterpret_cast<float4*>(reinterpret_cast<float*>(op) + d) =
                        make_float4(v4[0], v4[1], v4[2], v4[3]);
                } else {
                    *reinterpret_cast<uint2*>(reinterpret_cast<uint16_t*>(op) + d) =
                        make_uint2(pack_bf16x2(v4[0], v4[1]), pack_bf16x2(v4[2], v4[3]));
                }
            }
    }
}

}  // namespace
}  // namespace dit

namespace dit {
namespace {

// Shared checks of k, v, o, the sizes and the strides; q and its strides are
// checked only when given (the prologue takes its own).
int attn_prepare(const void* q, const void* k, const void* v, void* o, int64_t batch, int64_t heads,
                 int64_t seq_q, int64_t seq_kv, int64_t head_dim, const int64_t* q_strides,
                 const int64_t* k_strides, const int64_t* v_strides, const int64_t* o_strides, float scale,
                 int32_t o_type, const char* who, AttnArgs* out) {
    DT_REQUIRE(head_dim == D, "%s: head_dim %lld unsupported (128 only)", who, (long long)head_dim);
    DT_REQUIRE(o_type == DT_TYPE_BF16 || o_type == DT_TYPE_F32, "%s: o_type %d unsupported", who, o_type);
    DT_REQUIRE(batch >= 0 && heads >= 0 && seq_q >= 0 && seq_kv >= 0, "%s: negative size", who);
    DT_REQUIRE(seq_kv > 0 || batch == 0 || heads == 0 || seq_q == 0, "%s: seq_kv must be positive", who);
    DT_REQUIRE(k && v && o && k_strides && v_strides && o_strides && (!q || q_strides), "%s: null pointer", who);
    DT_REQUIRE(seq_q < (1ll << 30) && seq_kv < (1ll << 30) && heads < (1 << 20) && batch < (1 << 20),
               "%s: size too large", who);
    AttnArgs a{};
    a.q = (const uint16_t*)q;
    a.k = (const uint16_t*)k;
    a.v = (const uint16_t*)v;
    a.o = o;
    for (int i = 0; i < 3; ++i) {
        a.qs[i] = q ? q_strides[i] : 0;
        a.ks[i] = k_strides[i];
        a.vs[i] = v_strides[i];
        a.os[i] = o_strides[i];
        DT_REQUIRE(a.qs[i] % 8 == 0 && a.ks[i] % 8 == 0 && a.vs[i] % 8 == 0 && a.os[i] % 4 == 0,
                   "%s: strides must keep rows 16-byte aligned", who);
    }
    DT_REQUIRE((!q || aligned16(q)) && aligned16(k) && aligned16(v) && aligned16(o),
               "%s: pointers must be 16-byte aligned", who);
    a.batch = (int32_t)batch;
    a.heads = (int32_t)heads;
    a.seq_q = (int32_t)seq_q;
    a.seq_kv = (int32_t)seq_kv;
    a.q_blocks = (int32_t)((seq_q + QB - 1) / QB);
    DT_REQUIRE(scale >= 0.f, "%s: scale must be >= 0 (got %g)", who, (double)scale);
    a.scale_log2 = scale * 1.4426950408889634f;
    DT_REQUIRE((int64_t)a.q_blocks * heads * batch < (1ll << 31), "%s: grid too large", who);
    *out = a;
    return DT_OK;
}

template <bool PRO>
int attn_launch(const AttnArgs& a, const AttnPro& pro, int32_t o_type, hipStream_t st, const char* who) {
    const unsigned nblocks = (unsigned)((int64_t)a.q_blocks * a.heads * a.batch);
    if (nblocks == 0) return DT_OK;
    if (o_type == DT_TYPE_F32)
        hipLaunchKernelGGL((flash_attn_dma_kernel<float, PRO>), dim3(nblocks), dim3(256), 0, st, a, pro);
    else
        hipLaunchKernelGGL((flash_attn_dma_kernel<uint16_t, PRO>), dim3(nblocks), dim3(256), 0, st, a, pro);
    return check_launch(who);
}

}  // namespace

int flash_attn_qk_launch(const AttnQk& qk, const void* k, const void* v, void* o, int64_t batch, int64_t heads,
                         int64_t seq_q, int64_t seq_kv, const int64_t* k_strides, const int64_t* v_strides,
                         const int64_t* o_strides, float scale, int32_t o_type, hipStream_t st) {
    const char* who = "dt_flash_attn_qk_bf16";
    AttnArgs a;
    int rc = attn_prepare(nullptr, k, v, o, batch, heads, seq_q, seq_kv, D, nullptr, k_strides, v_strides,
                          o_strides, scale, o_type, who, &a);
    if (rc || a.q_blocks == 0 || heads == 0 || batch == 0) return rc;
    DT_REQUIRE(qk.n_axes > 0 && qk.n_axes <= kMaxRopeAxes && qk.axis_dim > 0 && qk.axis_dim % 8 == 0 &&
                   qk.n_axes * qk.axis_dim == D,
               "%s: need n_axes <= %d, axis_dim %% 8 == 0 and n_axes * axis_dim == 128 (%d * %d)", who,
               kMaxRopeAxes, qk.n_axes, qk.axis_dim);
    DT_REQUIRE(qk.split >= 0, "%s: split < 0", who);
    const bool two = qk.split < seq_q;
    DT_REQUIRE(qk.q[0] && qk.w[0] && (!two || (qk.q[1] && qk.w[1])), "%s: null q or norm weight", who);
    for (int sgi = 0; sgi < (two ? 2 : 1); ++sgi) {
        DT_REQUIRE(aligned16(qk.q[sgi]) && aligned16(qk.w[sgi]), "%s: q / weights must be 16-byte aligned", who);
        for (int i = 0; i < 3; ++i)
            DT_REQUIRE(qk.qs[sgi][i] % 8 == 0, "%s: q strides must keep rows 16-byte aligned", who);
    }
    for (int ax = 0; ax < qk.n_axes; ++ax)
        DT_REQUIRE(qk.pos.ptr[ax] != nullptr, "%s: null position pointer for axis %d", who, ax);
    DT_REQUIRE(!qk.table || (aligned16(qk.table) && qk.n_pos >= 0), "%s: rope table must be 16-byte aligned", who);
    AttnPro pro{};
    pro.q0 = (const uint16_t*)qk.q[0];
    pro.q0_bs = qk.qs[0][0];
    pro.q0_ts = qk.qs[0][1];
    pro.q0_hs = qk.qs[0][2];
    pro.w0 = qk.w[0];
    if (two) {
        pro.q1 = (const uint16_t*)qk.q[1];
        pro.q1_bs = qk.qs[1][0];
        pro.q1_ts = qk.qs[1][1];
        pro.q1_hs = qk.qs[1][2];
        pro.w1 = qk.w[1];
    }
    pro.split = (int32_t)std::min<int64_t>(qk.split, seq_q);
    pro.axis_dim = qk.axis_dim;
    pro.n_pos = qk.table ? qk.n_pos : 0;
    pro.theta_scale = powf(qk.freq_base, -2.0f / (float)qk.axis_dim);
    pro.eps = qk.eps;
    pro.table = qk.table;
    pro.pos = qk.pos;
    for (int ax = qk.n_axes; ax < kMaxRopeAxes; ++ax) {
        pro.pos.ptr[ax] = qk.pos.ptr[0];
        pro.pos.stride[ax] = qk.pos.stride[0];
    }
    a.q = pro.q0;
    return attn_launch<true>(a, pro, o_type, st, who);
}

}  // namespace dit

extern "C" int dt_flash_attn_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                  int64_t heads, int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                                  const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                                  const int64_t* o_strides, float scale, int32_t o_type, dt_stream_t stream) {
    using namespace dit;
    const char* who = "dt_flash_attn_bf16";
    DT_REQUIRE(head_dim == D, "%s: head_dim %lld unsupported (128 only)", who, (long long)head_dim);
    if (batch == 0 || heads == 0 || seq_q == 0) return DT_OK;
    DT_REQUIRE(q != nullptr, "%s: null pointer", who);
    AttnArgs a;
    int rc = attn_prepare(q, k, v, o, batch, heads, seq_q, seq_kv, head_dim, q_strides, k_strides, v_strides,
                          o_strides, scale, o_type, who, &a);
    if (rc) return rc;
    return attn_launch<false>(a, AttnPro{}, o_type, (hipStream_t)stream, who);
}

extern "C" int dt_flash_attn_qk_bf16(const void* q0, const int64_t* q0_strides, const float* w0, const void* q1,
                                     const int64_t* q1_strides, const float* w1, int64_t split, float eps,
                                     const int32_t* pos, int64_t pos_stride, int32_t n_axes, int32_t axis_dim,
                                     float freq_base, const float* rope_table, int32_t n_pos, const void* k,
                                     const void* v, void* o, int64_t batch, int64_t heads, int64_t seq_q,
                                     int64_t seq_kv, int64_t head_dim, const int64_t* k_strides,
                                     const int64_t* v_strides, const int64_t* o_strides, float scale,
                                     int32_t o_type, dt_stream_t stream) {
    using namespace dit;
    const char* who = "dt_flash_attn_qk_bf16";
    DT_REQUIRE(head_dim == D, "%s: head_dim %lld unsupported (128 only)", who, (long long)head_dim);
    if (batch == 0 || heads == 0 || seq_q == 0) return DT_OK;
    DT_REQUIRE(q0_strides && (split >= seq_q || q1_strides), "%s: null q strides", who);
    DT_REQUIRE(pos != nullptr && pos_stride >= n_axes && n_axes > 0 && n_axes <= kMaxRopeAxes,
               "%s: bad positions (pos_stride %lld, n_axes %d)", who, (long long)pos_stride, n_axes);
    AttnQk qk{};
    qk.q[0] = q0;
    qk.q[1] = q1;
    qk.w[0] = w0;
    qk.w[1] = w1;
    for (int i = 0; i < 3; ++i) {
        qk.qs[0][i] = q0_strides[i];
        qk.qs[1][i] = split < seq_q ? q1_strides[i] : 0;
    }
    qk.split = split;
    qk.eps = eps;
    for (int ax = 0; ax < n_axes; ++ax) {
        qk.pos.ptr[ax] = pos + ax;
        qk.pos.stride[ax] = pos_stride;
    }
    qk.n_axes = n_axes;
    qk.axis_dim = axis_dim;
    qk.freq_base = freq_base;
    qk.table = n_pos > 0 ? rope_table : nullptr;
    qk.n_pos = n_pos;
    return flash_attn_qk_launch(qk, k, v, o, batch, heads, seq_q, seq_kv, k_strides, v_strides, o_strides, scale,
                                o_type, (hipStream_t)stream);
}
