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
// in LDS; V is stored transposed (Vt[d][key]) so the A operand is two 8-byte
// LDS reads.  The next tile is fetched into registers while the MFMAs run.
// Workgroups are ordered so that each XCD (8 per MI355X, one L2 each) works
// through a contiguous range of (batch, head) slices.
#include "capi_util.hpp"
#include "common.hpp"

namespace dit {
namespace {

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int D = 128;       // head dim
constexpr int QB = 128;      // queries per workgroup
constexpr int KB = 64;       // keys per tile
constexpr int KS = D + 8;    // Ks row, bf16 elements (272 B: conflict-free 16-byte reads)
constexpr int VS = KB + 4;   // Vt row, bf16 elements (136 B: conflict-free 8-byte reads)

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

__device__ __forceinline__ uint4 ld16(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

template <typename TO>
__global__ __launch_bounds__(256) void flash_attn_d128_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t Ks[KB * KS];
    __shared__ __attribute__((aligned(16))) uint16_t Vt[D * VS];

    // XCD-aware order: workgroup i runs on XCD i % 8; give each XCD a
    // contiguous range of logical tiles so (batch, head) slices stay in one L2.
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

    // Q^T as the B operand of S^T = K Q^T: lane (r, g) holds Q[q0 + r][16 c + 8 g .. +8].
    bf16x8_t qf[8];
    {
        const int qrow = q0 + r;
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            uint4 u = qrow < a.seq_q ? ld16(Qp + (int64_t)qrow * a.qs[1] + 16 * c + 8 * g) : make_uint4(0, 0, 0, 0);
            qf[c] = __builtin_bit_cast(bf16x8_t, u);
        }
    }

    // Tile fetch: K rows are 16 threads x 16 bytes; V is fetched as key pairs
    // (2p, 2p+1) of one 8-wide d chunk so the transposed LDS store packs two
    // keys per 32-bit word.
    uint4 kr[4], vr[2][2];
    auto fetch = [&](int kv0) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 256 * i, key = c >> 4, ch = c & 15;
            kr[i] = kv0 + key < a.seq_kv ? ld16(Kp + (int64_t)(kv0 + key) * a.ks[1] + ch * 8)
                                         : make_uint4(0, 0, 0, 0);
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int p = tid & 31, ch = (tid >> 5) + 8 * j;
#pragma unroll
            for (int e = 0; e < 2; ++e) {
                const int key = kv0 + 2 * p + e;
                vr[j][e] = key < a.seq_kv ? ld16(Vp + (int64_t)key * a.vs[1] + ch * 8) : make_uint4(0, 0, 0, 0);
            }
        }
    };
    auto stash = [&]() {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int c = tid + 256 * i, key = c >> 4, ch = c & 15;
            *reinterpret_cast<uint4*>(&Ks[key * KS + ch * 8]) = kr[i];
        }
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int p = tid & 31, ch = (tid >> 5) + 8 * j;
            const uint32_t* lo = reinterpret_cast<const uint32_t*>(&vr[j][0]);
            const uint32_t* hi = reinterpret_cast<const uint32_t*>(&vr[j][1]);
#pragma unroll
            for (int w = 0; w < 4; ++w) {
                // d = 8 ch + 2 w (+1): low / high halves of word w of each key's chunk
                const uint32_t d0 = (lo[w] & 0xFFFFu) | (hi[w] << 16);
                const uint32_t d1 = (lo[w] >> 16) | (hi[w] & 0xFFFF0000u);
                *reinterpret_cast<uint32_t*>(&Vt[(8 * ch + 2 * w) * VS + 2 * p]) = d0;
                *reinterpret_cast<uint32_t*>(&Vt[(8 * ch + 2 * w + 1) * VS + 2 * p]) = d1;
            }
        }
    };

    f32x16_t o[4];
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
        for (int e = 0; e < 16; ++e) o[t][e] = 0.f;
    float m_run = -INFINITY, l_run = 0.f;

    fetch(0);
    for (int kv0 = 0; kv0 < a.seq_kv; kv0 += KB) {
        stash();
        __syncthreads();
        if (kv0 + KB < a.seq_kv) fetch(kv0 + KB);

        // S^T[key][q] for the two 32-key halves of the tile.
        f32x16_t s[2];
#pragma unroll
        for (int hh = 0; hh < 2; ++hh) {
#pragma unroll
            for (int e = 0; e < 16; ++e) s[hh][e] = 0.f;
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const bf16x8_t kf = *reinterpret_cast<const bf16x8_t*>(&Ks[(32 * hh + r) * KS + 16 * c + 8 * g]);
                s[hh] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[c], s[hh], 0, 0, 0);
            }
        }

        // Online softmax for query q0 + r; element i of s[hh] is key
        // kv0 + 32 hh + 8 (i / 4) + 4 g + i % 4.
        float mx = -INFINITY;
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int key = kv0 + 32 * hh + 8 * (i >> 2) + 4 * g + (i & 3);
                float t = s[hh][i] * a.scale_log2;
                if (key >= a.seq_kv) t = -INFINITY;
                s[hh][i] = t;
                mx = fmaxf(mx, t);
            }
        mx = fmaxf(mx, __shfl_xor(mx, 32));
        const float m_new = fmaxf(m_run, mx);
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        m_run = m_new;
        float psum = 0.f;
        bf16x8_t pf[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const float p = __builtin_amdgcn_exp2f(s[j >> 1][8 * (j & 1) + e] - m_new);
                psum += p;
                pf[j][e] = (__bf16)p;
            }
        }
        l_run = l_run * alpha + psum;
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[t][e] *= alpha;

        // O^T[d][q] += V^T[d][key] P^T[key][q], 16 keys per MFMA.
#pragma unroll
        for (int j = 0; j < 4; ++j) {
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                const uint16_t* vrow = &Vt[(32 * t + r) * VS + 16 * j + 4 * g];
                const uint2 lo = *reinterpret_cast<const uint2*>(vrow);
                const uint2 hi = *reinterpret_cast<const uint2*>(vrow + 8);
                const bf16x8_t vf = __builtin_bit_cast(bf16x8_t, make_uint4(lo.x, lo.y, hi.x, hi.y));
                o[t] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[j], o[t], 0, 0, 0);
            }
        }
        __syncthreads();
    }

    // Normalise and store O[q][d]: element i of o[t] is d = 32 t + 8 (i / 4) + 4 g + i % 4.
    const float l_tot = l_run + __shfl_xor(l_run, 32);
    const float inv = 1.0f / l_tot;
    const int q = q0 + r;
    if (q < a.seq_q) {
        TO* op = reinterpret_cast<TO*>(a.o) + b * a.os[0] + (int64_t)q * a.os[1] + h * a.os[2];
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
            for (int i4 = 0; i4 < 4; ++i4) {
                const int d = 32 * t + 8 * i4 + 4 * g;
                float v4[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v4[e] = o[t][4 * i4 + e] * inv;
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

extern "C" int dt_flash_attn_bf16(const void* q, const void* k, const void* v, void* o, int64_t batch,
                                  int64_t heads, int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                                  const int64_t* q_strides, const int64_t* k_strides, const int64_t* v_strides,
                                  const int64_t* o_strides, float scale, int32_t o_type, dt_stream_t stream) {
    DT_REQUIRE(head_dim == dit::D, "dt_flash_attn_bf16: head_dim %lld unsupported (128 only)", (long long)head_dim);
    DT_REQUIRE(o_type == DT_TYPE_BF16 || o_type == DT_TYPE_F32, "dt_flash_attn_bf16: o_type %d unsupported", o_type);
    DT_REQUIRE(batch >= 0 && heads >= 0 && seq_q >= 0 && seq_kv >= 0, "dt_flash_attn_bf16: negative size");
    if (batch == 0 || heads == 0 || seq_q == 0) return DT_OK;
    DT_REQUIRE(seq_kv > 0, "dt_flash_attn_bf16: seq_kv must be positive");
    DT_REQUIRE(q && k && v && o && q_strides && k_strides && v_strides && o_strides,
               "dt_flash_attn_bf16: null pointer");
    DT_REQUIRE(seq_q < (1ll << 30) && seq_kv < (1ll << 30) && heads < (1 << 20) && batch < (1 << 20),
               "dt_flash_attn_bf16: size too large");
    dit::AttnArgs a{};
    a.q = (const uint16_t*)q;
    a.k = (const uint16_t*)k;
    a.v = (const uint16_t*)v;
    a.o = o;
    for (int i = 0; i < 3; ++i) {
        a.qs[i] = q_strides[i];
        a.ks[i] = k_strides[i];
        a.vs[i] = v_strides[i];
        a.os[i] = o_strides[i];
        DT_REQUIRE(a.qs[i] % 8 == 0 && a.ks[i] % 8 == 0 && a.vs[i] % 8 == 0 && a.os[i] % 4 == 0,
                   "dt_flash_attn_bf16: strides must keep rows 16-byte aligned");
    }
    DT_REQUIRE(dit::aligned16(q) && dit::aligned16(k) && dit::aligned16(v) && dit::aligned16(o),
               "dt_flash_attn_bf16: pointers must be 16-byte aligned");
    a.batch = (int32_t)batch;
    a.heads = (int32_t)heads;
    a.seq_q = (int32_t)seq_q;
    a.seq_kv = (int32_t)seq_kv;
    a.q_blocks = (int32_t)((seq_q + dit::QB - 1) / dit::QB);
    a.scale_log2 = scale * 1.4426950408889634f;
    const int64_t nblocks = (int64_t)a.q_blocks * heads * batch;
    DT_REQUIRE(nblocks < (1ll << 31), "dt_flash_attn_bf16: grid too large");
    hipStream_t st = (hipStream_t)stream;
    if (o_type == DT_TYPE_F32)
        hipLaunchKernelGGL((dit::flash_attn_d128_kernel<float>), dim3((unsigned)nblocks), dim3(256), 0, st, a);
    else
        hipLaunchKernelGGL((dit::flash_attn_d128_kernel<uint16_t>), dim3((unsigned)nblocks), dim3(256), 0, st, a);
    return dit::check_launch("dt_flash_attn_bf16");
}
