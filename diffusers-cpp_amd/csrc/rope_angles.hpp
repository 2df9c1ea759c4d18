// rope_angles.hpp -- cos/sin of RoPE NORMAL-mode pairs, shared by the
// QK-RMSNorm+RoPE kernels (qk_rope.hip) and the attention Q prologue
// (attention.hip), so both produce the same bits for the same position.
// ggml's angle for pair k of an axis of n_dims at position p is the fp32
// recurrence theta_0 = p, theta_{k+1} = theta_k * freq_base^(-2/n_dims)
// (rope_ext, Runtime.hpp:281-293; Flux2PosEmbed.hpp:79-95).
#pragma once

#include "common.hpp"

namespace dit {
namespace {

// cos/sin of pairs [i0/2, i0/2 + NP) of an axis at position p, interleaved
// (cos, sin) in cs[2 NP]: from the table row p when p is inside it, else by
// the recurrence on the device.
template <int NP>
__device__ __forceinline__ void rope_angles(int p, int i0, const float* __restrict__ table,
                                            int n_pos, int axis_dim, float theta_scale,
                                            float* cs) {
    if (table != nullptr && p >= 0 && p < n_pos) {
        const float* t = table + (int64_t)p * axis_dim + i0;
#pragma unroll
        for (int e = 0; e < 2 * NP; e += 4) {
            const float4 a = *reinterpret_cast<const float4*>(t + e);
            cs[e] = a.x; cs[e + 1] = a.y; cs[e + 2] = a.z; cs[e + 3] = a.w;
        }
    } else {
        // Same fp32 recurrence as the table: theta_0 = p, theta *= scale.
        float theta = (float)p;
        for (int k = 0; k < i0 / 2; ++k) theta = mul_rn(theta, theta_scale);
#pragma unroll
        for (int q = 0; q < NP; ++q) {
            cs[2 * q] = cosf(theta);
            cs[2 * q + 1] = sinf(theta);
            theta = mul_rn(theta, theta_scale);
        }
    }
}

}  // namespace
}  // namespace dit
