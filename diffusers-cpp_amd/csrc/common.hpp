// common.hpp -- shared device helpers for the gfx950 kernels: bf16 bit
// conversions, 128-bit vector I/O over fp32/bf16 rows, wave64 reductions
// built on DPP row operations, and a 32-bit invariant-divisor helper.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dit_hip.h"

namespace dit {

constexpr int kWave = 64;

// bf16 as a distinct type so templates can tell it apart from uint16_t data.
struct bf16 {
    uint16_t bits;
};

__device__ __forceinline__ float bf16_lo(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t w) { return __uint_as_float(w & 0xFFFF0000u); }

// Round-to-nearest-even fp32 -> bf16 by gfx950's packed convert
// (v_cvt_pk_bf16_f32): ties to even, a NaN keeps its upper payload bits with
// the quiet bit set -- (u >> 16) | 0x40, ggml's fp32 -> bf16 rule.  Checked
// bit for bit against that integer formulation over all 2^32 fp32 patterns,
// in both halves of the pair.
typedef float f32x2_cvt __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_cvt __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2_cvt v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_cvt));
}

__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) { return pack_bf16x2(f, 0.f) & 0xFFFFu; }

// The same rounding in integer arithmetic (the reference formulation the
// hardware convert is checked against).
__device__ __forceinline__ uint32_t f32_to_bf16_bits_int(float f) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7FFFFFFFu) > 0x7F800000u) return (u >> 16) | 0x40u;
    return (u + 0x7FFFu + ((u >> 16) & 1u)) >> 16;
}

__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Round-to-nearest-even fp32 -> fp16 bits.
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// 16-byte non-temporal (streaming) global accesses.  Activations are read
// once and written once, so they bypass cache allocation; on gfx950 this
// nearly doubles sustained HBM bandwidth of read+write streams compared with
// default-policy accesses (measured on a 2-in/1-out 255 MB stream: ~6.0 vs
// ~3.3 TB/s).  Small operands shared by many lanes (modulation vectors, norm
// weights, RoPE tables) keep default-policy loads so they stay cached.
typedef unsigned int v4u __attribute__((ext_vector_type(4)));

__device__ __forceinline__ uint4 ld_stream(const void* p) {
    const v4u v = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(v.x, v.y, v.z, v.w);
}

__device__ __forceinline__ void st_stream(void* p, uint4 v) {
    const v4u t = {v.x, v.y, v.z, v.w};
    __builtin_nontemporal_store(t, reinterpret_cast<v4u*>(p));
}

// x / (1 + 2^(-x log2 e)) with the hardware exp2 and reciprocal (GroupNorm's
// SiLU, wherever it is applied).  Large negative x: the exponential
// overflows to inf and the result is -0.
__device__ __forceinline__ float silu_fast(float t) {
    const float e = __builtin_amdgcn_exp2f(t * -1.4426950408889634f);
    return t * __builtin_amdgcn_rcpf(1.0f + e);
}

// Row I/O in 16-byte vectors (streaming policy).  EPV = elements per vector.
template <typename T> struct Io;

template <> struct Io<float> {
    static constexpr int EPV = 4;
    static constexpr int kType = DT_TYPE_F32;
    __device__ __forceinline__ static void load(const float* p, float* v) {
        const uint4 t = ld_stream(p);
        v[0] = __uint_as_float(t.x); v[1] = __uint_as_float(t.y);
        v[2] = __uint_as_float(t.z); v[3] = __uint_as_float(t.w);
    }
    __device__ __forceinline__ static void store(float* p, const float* v) {
        st_stream(p, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                                __float_as_uint(v[3])));
    }
    __device__ __forceinline__ static float get(const float* p) { return *p; }
    __device__ __forceinline__ static void put(float* p, float v) { *p = v; }
    __device__ __forceinline__ static void unpack(uint4 t, float* v) {
        v[0] = __uint_as_float(t.x); v[1] = __uint_as_float(t.y);
        v[2] = __uint_as_float(t.z); v[3] = __uint_as_float(t.w);
    }
    // The values the type stores (identity for fp32).
    __device__ __forceinline__ static void round(float*) {}
    // One 16-byte vector of stored values from EPV floats.
    __device__ __forceinline__ static uint4 pack(const float* v) {
        return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3]));
    }
};

template <> struct Io<bf16> {
    static constexpr int EPV = 8;
    static constexpr int kType = DT_TYPE_BF16;
    __device__ __forceinline__ static void load(const bf16* p, float* v) {
        const uint4 t = ld_stream(p);
        v[0] = bf16_lo(t.x); v[1] = bf16_hi(t.x);
        v[2] = bf16_lo(t.y); v[3] = bf16_hi(t.y);
        v[4] = bf16_lo(t.z); v[5] = bf16_hi(t.z);
        v[6] = bf16_lo(t.w); v[7] = bf16_hi(t.w);
    }
    __device__ __forceinline__ static void store(bf16* p, const float* v) {
        uint4 t;
        t.x = pack_bf16x2(v[0], v[1]);
        t.y = pack_bf16x2(v[2], v[3]);
        t.z = pack_bf16x2(v[4], v[5]);
        t.w = pack_bf16x2(v[6], v[7]);
        st_stream(p, t);
    }
    __device__ __forceinline__ static float get(const bf16* p) { return __uint_as_float((uint32_t)p->bits << 16); }
    __device__ __forceinline__ static void put(bf16* p, float v) { p->bits = (uint16_t)f32_to_bf16_bits(v); }
    __device__ __forceinline__ static void unpack(uint4 t, float* v) {
        v[0] = bf16_lo(t.x); v[1] = bf16_hi(t.x);
        v[2] = bf16_lo(t.y); v[3] = bf16_hi(t.y);
        v[4] = bf16_lo(t.z); v[5] = bf16_hi(t.z);
        v[6] = bf16_lo(t.w); v[7] = bf16_hi(t.w);
    }
    __device__ __forceinline__ static uint4 pack(const float* v) {
        return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                          pack_bf16x2(v[6], v[7]));
    }
    // The values the type stores: RNE to bf16 and back.
    __device__ __forceinline__ static void round(float* v) {
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
            const uint32_t t = pack_bf16x2(v[e], v[e + 1]);
            v[e] = bf16_lo(t);
            v[e + 1] = bf16_hi(t);
        }
    }
};

// Explicitly rounded fp32 arithmetic: keeps the compiler from contracting
// a*b+c into one fma where the emitted ggml graph rounds after each op.
__device__ __forceinline__ float mul_rn(float a, float b) { return __fmul_rn(a, b); }
__device__ __forceinline__ float add_rn(float a, float b) { return __fadd_rn(a, b); }
__device__ __forceinline__ float sub_rn(float a, float b) { return __fsub_rn(a, b); }

// ggml's sigmoid, 1/(1+expf(-x)), with the accurate device expf.
__device__ __forceinline__ float sigmoid_ref(float x) { return 1.0f / (1.0f + expf(-x)); }

// ---- DPP-based reductions ---------------------------------------------------
// dpp_ctrl encodings (GCN/CDNA): quad_perm = p0 | p1<<2 | p2<<4 | p3<<6,
// row_mirror = 0x140, row_half_mirror = 0x141.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Sum across each 16-lane DPP row; every lane of the row receives the sum.
__device__ __forceinline__ float row16_sum(float v) {
    v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]: lane ^ 1
    v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]: lane ^ 2
    v += dpp_f32<0x141>(v);  // row_half_mirror: pairs quad 0 with quad 1
    v += dpp_f32<0x140>(v);  // row_mirror: pairs the two halves of the row
    return v;
}

// Sum across the full wave64; every lane receives the sum.
__device__ __forceinline__ float wave_sum(float v) {
    v = row16_sum(v);
    v += __shfl_xor(v, 16, kWave);
    v += __shfl_xor(v, 32, kWave);
    return v;
}

__device__ __forceinline__ double wave_sum_f64(double v) {
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
    return v;
}

// Block-wide sum of doubles through LDS; `red` holds >= blockDim.x/64 slots.
// All threads receive the result.  Must be called by every thread.
__device__ __forceinline__ double block_sum_f64(double v, double* red) {
    v = wave_sum_f64(v);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int nw = (blockDim.x + kWave - 1) / kWave;
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    double s = 0.0;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

// Two block_sum_f64 at once, with the same sums in the same order (so the
// same bits), through one LDS exchange: red2 holds 2 doubles per wave.
__device__ __forceinline__ void block_sum2_f64(double& a, double& b, double* red2) {
    a = wave_sum_f64(a);
    b = wave_sum_f64(b);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int nw = (blockDim.x + kWave - 1) / kWave;
    __syncthreads();
    if (lane == 0) {
        red2[2 * wid] = a;
        red2[2 * wid + 1] = b;
    }
    __syncthreads();
    a = 0.0;
    b = 0.0;
    for (int i = 0; i < nw; ++i) {
        a += red2[2 * i];
        b += red2[2 * i + 1];
    }
}

__device__ __forceinline__ float block_sum_f32(float v, float* red) {
    v = wave_sum(v);
    const int lane = threadIdx.x & (kWave - 1), wid = threadIdx.x / kWave;
    const int nw = (blockDim.x + kWave - 1) / kWave;
    __syncthreads();
    if (lane == 0) red[wid] = v;
    __syncthreads();
    float s = 0.0f;
    for (int i = 0; i < nw; ++i) s += red[i];
    return s;
}

// ---- invariant 32-bit division (n < 2^31) -----------------------------------
struct FastDiv {
    uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
    FastDiv f;
    f.d = d;
    uint32_t l = 0;
    while ((1ull << l) < d) ++l;
    f.s = l;
    f.m = (uint32_t)(((1ull << 32) * ((1ull << l) - d)) / d + 1);
    return f;
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
    return (__umulhi(n, f.m) + n) >> f.s;
}

}  // namespace dit
