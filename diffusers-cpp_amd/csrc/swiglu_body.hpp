// swiglu_body.hpp -- the SwiGLU streaming body, y = (g * sigmoid(g)) * u
// (Flux2SwiGLU.hpp:17-21, SiLU.hpp:9-13), shared by the standalone kernel
// (elementwise.hip) and the launch that runs it beside the QK-RMSNorm+RoPE
// of the same block (qk_rope.hip).  A workgroup of B threads moves U
// 16-byte vectors per thread and operand: all loads before any math,
// non-temporal accesses, consecutive threads on consecutive vectors, the row
// of a vector from a multiply-high invariant division.  One vector per
// thread in 512-thread workgroups streams fastest on gfx950 at [4608, 9216]
// (42.4 us cold vs 44.4-50.2 us for 2 or 4 vectors, or for 256/1024 threads).
#pragma once

#include "common.hpp"

namespace dit {

struct SwigluArgs {
    const void* g;
    int64_t gs;
    const void* u;
    int64_t us;
    void* y;
    int64_t ys;
    uint32_t total;  // 16-byte vectors in the output
    FastDiv nv;      // vectors per row
};

constexpr int kSwigluUnroll = 1;

template <typename T, int B>
__device__ __forceinline__ void swiglu_body(const SwigluArgs& a, int block) {
    constexpr int EPV = Io<T>::EPV, U = kSwigluUnroll;
    const T* __restrict__ g = (const T*)a.g;
    const T* __restrict__ u = (const T*)a.u;
    T* __restrict__ y = (T*)a.y;
    const uint32_t base = (uint32_t)block * (B * U) + threadIdx.x;
    float gv[U][EPV], uv[U][EPV];
    int64_t yo[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
        const uint32_t idx = base + k * B;
        yo[k] = -1;
        if (idx < a.total) {
            const uint32_t r = fdiv(idx, a.nv);
            const uint32_t c = (idx - r * a.nv.d) * EPV;
            Io<T>::load(g + r * a.gs + c, gv[k]);
            Io<T>::load(u + r * a.us + c, uv[k]);
            yo[k] = r * a.ys + c;
        }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
        if (yo[k] >= 0) {
            float o[EPV];
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                const float s = sigmoid_ref(gv[k][e]);
                o[e] = mul_rn(mul_rn(gv[k][e], s), uv[k][e]);
            }
            Io<T>::store(y + yo[k], o);
        }
    }
}

// Workgroups of B threads that cover a SwiGLU.
template <typename T, int B>
inline int64_t swiglu_blocks(uint32_t total) {
    return ((int64_t)total + B * kSwigluUnroll - 1) / (B * kSwigluUnroll);
}

}  // namespace dit
