// adaln.hip -- fused LayerNorm(no affine) + adaLN modulation:
//   y = add(mul(norm_eps(x), add(scale, 1.0f)), shift)
// the node chain LayerNorm::forward + `(1 + scale) * n + shift` emits in
// Flux2SingleTransformerBlock.hpp:50-54 / Flux2TransformerBlock.hpp:63-72.
//
// Fast path: one wave64 per row.  The row is held in VGPRs as its raw
// 16-byte vectors (bf16 stays packed: 24 VGPRs for 3072 columns) with all of
// its loads issued back to back and each value unpacked where it is used;
// the mean and the centred variance are two wave-wide DPP reductions, and
// while the row loads are in flight each workgroup stages the fp32
// (1 + scale, shift) vectors, shared by every row, into LDS (24 KB at 3072
// columns).  Registers and LDS are sized so that every row of a Flux2
// activation ([4608, 3072]) is resident at once: a row that waits for a
// second round of workgroups costs a full memory latency at the tail.
#include "capi_util.hpp"
#include "common.hpp"
#include "kernels.hpp"

namespace dit {
namespace {

template <typename T, int VPL, bool FULL, int WPB>
__global__ __launch_bounds__(WPB * kWave) void adaln_wave_kernel(
    const T* __restrict__ x, int64_t xs, const float* __restrict__ shift,
    const float* __restrict__ scale, T* __restrict__ y, int64_t ys, int rows,
    int nvec, float cols_f, float eps, float addend) {
    constexpr int EPV = Io<T>::EPV;
    // (scale + addend, shift) interleaved per 4 columns: [nvec * EPV / 4][8].
    extern __shared__ float4 mod_lds[];
    const int lane = threadIdx.x & (kWave - 1);
    const int r = (int)(blockIdx.x * WPB + threadIdx.x / kWave);
    const bool active = r < rows;
    const T* xr = x + (int64_t)r * xs;
    T* yr = y + (int64_t)r * ys;

    // The whole row is in flight at once: VPL independent 16-byte loads.
    uint4 raw[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int vi = lane + kWave * j;
        raw[j] = make_uint4(0, 0, 0, 0);
        if (active && (FULL || vi < nvec)) raw[j] = ld_stream(xr + (int64_t)vi * EPV);
    }
    // Meanwhile the workgroup stages the modulation vectors (L2 hits) in LDS.
    const int n4 = nvec * EPV / 4;
    for (int i = threadIdx.x; i < n4; i += WPB * kWave) {
        float4 sc = reinterpret_cast<const float4*>(scale)[i];
        sc.x += addend; sc.y += addend; sc.z += addend; sc.w += addend;
        mod_lds[2 * i] = sc;
        mod_lds[2 * i + 1] = reinterpret_cast<const float4*>(shift)[i];
    }
    __syncthreads();
    if (!active) return;
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        float v[EPV];
        Io<T>::unpack(raw[j], v);
#pragma unroll
        for (int e = 0; e < EPV; ++e) s += v[e];
    }
    s = wave_sum(s);
    const float mean = s / cols_f;
    float s2 = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        if (FULL || lane + kWave * j < nvec) {
            float v[EPV];
            Io<T>::unpack(raw[j], v);
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                const float d = v[e] - mean;
                s2 += d * d;
            }
        }
    }
    s2 = wave_sum(s2);
    const float rstd = 1.0f / sqrtf(s2 / cols_f + eps);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int vi = lane + kWave * j;
        if (FULL || vi < nvec) {
            float v[EPV], o[EPV];
            Io<T>::unpack(raw[j], v);
#pragma unroll
            for (int e = 0; e < EPV; e += 4) {
                const int i4 = (vi * EPV + e) / 4;
                const float4 t = mod_lds[2 * i4], sh = mod_lds[2 * i4 + 1];
                o[e + 0] = add_rn(mul_rn(mul_rn(v[e + 0] - mean, rstd), t.x), sh.x);
                o[e + 1] = add_rn(mul_rn(mul_rn(v[e + 1] - mean, rstd), t.y), sh.y);
                o[e + 2] = add_rn(mul_rn(mul_rn(v[e + 2] - mean, rstd), t.z), sh.z);
                o[e + 3] = add_rn(mul_rn(mul_rn(v[e + 3] - mean, rstd), t.w), sh.w);
            }
            st_stream(yr + (int64_t)vi * EPV, Io<T>::pack(o));
        }
    }
}

// Gated residual feeding the next adaLN, in one pass over the row:
//   r = h + gate * o           (Flux2SingleTransformerBlock.hpp:58, Flux2TransformerBlock.hpp:86-87, 100-101)
//   y = (1 + scale) * LayerNorm(r) + shift   (the next block's adaLN, :50-54 / :91-92)
// r is rounded to the I/O type before it is normalised, exactly as the
// unfused graph stores the ADD node and the NORM node reads it back.  One
// wave per row; h and o arrive as raw vectors and are replaced by the stored
// r (for bf16 the stored bits are exactly the rounded value); (gate,
// 1 + scale, shift) are staged in LDS per workgroup, 12 bytes per column.
template <typename T, int VPL, bool FULL>
__device__ __forceinline__ void residual_adaln_row(uint4 (&hr)[VPL], const uint4 (&orw)[VPL],
                                                   const float4* __restrict__ mod, int lane, int nvec, T* rr,
                                                   T* yr, float cols_f, float eps) {
    constexpr int EPV = Io<T>::EPV;
    // r = h + (o * gate), stored; its stored bits replace h in registers.
    float s = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int vi = lane + kWave * j;
        if (FULL || vi < nvec) {
            float hv[EPV], ov[EPV];
            Io<T>::unpack(hr[j], hv);
            Io<T>::unpack(orw[j], ov);
#pragma unroll
            for (int e = 0; e < EPV; e += 4) {
                const float4 g = mod[3 * ((vi * EPV + e) / 4)];
                hv[e + 0] = add_rn(hv[e + 0], mul_rn(ov[e + 0], g.x));
                hv[e + 1] = add_rn(hv[e + 1], mul_rn(ov[e + 1], g.y));
                hv[e + 2] = add_rn(hv[e + 2], mul_rn(ov[e + 2], g.z));
                hv[e + 3] = add_rn(hv[e + 3], mul_rn(ov[e + 3], g.w));
            }
            hr[j] = Io<T>::pack(hv);
            st_stream(rr + (int64_t)vi * EPV, hr[j]);
            Io<T>::unpack(hr[j], hv);
#pragma unroll
            for (int e = 0; e < EPV; ++e) s += hv[e];
        }
    }
    s = wave_sum(s);
    const float mean = s / cols_f;
    float s2 = 0.f;
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        if (FULL || lane + kWave * j < nvec) {
            float v[EPV];
            Io<T>::unpack(hr[j], v);
#pragma unroll
            for (int e = 0; e < EPV; ++e) {
                const float d = v[e] - mean;
                s2 += d * d;
            }
        }
    }
    s2 = wave_sum(s2);
    const float rstd = 1.0f / sqrtf(s2 / cols_f + eps);
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int vi = lane + kWave * j;
        if (FULL || vi < nvec) {
            float v[EPV], out[EPV];
            Io<T>::unpack(hr[j], v);
#pragma unroll
            for (int e = 0; e < EPV; e += 4) {
                const int i4 = (vi * EPV + e) / 4;
                const float4 t = mod[3 * i4 + 1], sh = mod[3 * i4 + 2];
                out[e + 0] = add_rn(mul_rn(mul_rn(v[e + 0] - mean, rstd), t.x), sh.x);
                out[e + 1] = add_rn(mul_rn(mul_rn(v[e + 1] - mean, rstd), t.y), sh.y);
                out[e + 2] = add_rn(mul_rn(mul_rn(v[e + 2] - mean, rstd), t.z), sh.z);
                out[e + 3] = add_rn(mul_rn(mul_rn(v[e + 3] - mean, rstd), t.w), sh.w);
            }
            st_stream(yr + (int64_t)vi * EPV, Io<T>::pack(out));
        }
    }
}

// (gate, scale + addend, shift) per 4 columns into LDS, by the whole workgroup.
__device__ __forceinline__ void stage_residual_mod(float4* mod_lds, const float* gate, const float* scale,
                                                   const float* shift, float addend, int n4, int threads) {
    for (int i = threadIdx.x; i < n4; i += threads) {
        float4 sc = reinterpret_cast<const float4*>(scale)[i];
        sc.x += addend; sc.y += addend; sc.z += addend; sc.w += addend;
        mod_lds[3 * i] = reinterpret_cast<const float4*>(gate)[i];
        mod_lds[3 * i + 1] = sc;
        mod_lds[3 * i + 2] = reinterpret_cast<const float4*>(shift)[i];
    }
}

// Every row resident at once: 36 KB of LDS at 3072 columns, so six rows per
// workgroup keep 4608 rows resident.  Measured on gfx950 at [4608, 3072]
// bf16: the bound of six waves per SIMD (80 VGPRs, 9 of them spilled) runs
// 4-6% faster than a bound of five (79 VGPRs, no spill); a persistent
// variant in which each wave walks several rows and prefetches the next
// row's h and o ran 25% slower, and 30% slower inside the Flux2 step.
template <typename T, int VPL, bool FULL, int WPB>
__global__ __launch_bounds__(WPB * kWave, FULL && VPL <= 6 ? 6 : 1) void residual_adaln_kernel(
    const T* __restrict__ h, int64_t hs, const T* __restrict__ o, int64_t os, const float* __restrict__ gate,
    T* __restrict__ r_out, int64_t rs, const float* __restrict__ shift, const float* __restrict__ scale,
    T* __restrict__ y, int64_t ys, int rows, int nvec, float cols_f, float eps, float addend) {
    constexpr int EPV = Io<T>::EPV;
    extern __shared__ float4 mod_lds[];  // per 4 columns: (gate, scale + addend, shift)
    const int lane = threadIdx.x & (kWave - 1);
    const int row = (int)(blockIdx.x * WPB + threadIdx.x / kWave);
    const bool active = row < rows;

    uint4 hr[VPL], orw[VPL];
#pragma unroll
    for (int j = 0; j < VPL; ++j) {
        const int vi = lane + kWave * j;
        hr[j] = orw[j] = make_uint4(0, 0, 0, 0);
        if (active && (FULL || vi < nvec)) {
            hr[j] = ld_stream(h + (int64_t)row * hs + (int64_t)vi * EPV);
            orw[j] = ld_stream(o + (int64_t)row * os + (int64_t)vi * EPV);
        }
    }
    stage_residual_mod(mod_lds, gate, scale, shift, addend, nvec * EPV / 4, WPB * kWave);
    __syncthreads();
    if (!active) return;
    residual_adaln_row<T, VPL, FULL>(hr, orw, mod_lds, lane, nvec, r_out + (int64_t)row * rs, y + (int64_t)row * ys,
                                     cols_f, eps);
}

// Any cols / stride / alignment: one 256-thread block per row, LDS reductions.
template <typename T>
__global__ __launch_bounds__(256) void adaln_generic_kernel(
    const T* __restrict__ x, int64_t xs, const float* __restrict__ shift,
    const float* __restrict__ scale, T* y, int64_t ys, int64_t cols, float eps, float addend) {
    __shared__ float red[4];
    const T* xr = x + (int64_t)blockIdx.x * xs;
    T* yr = y + (int64_t)blockIdx.x * ys;
    float s = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) s += Io<T>::get(xr + c);
    const float mean = block_sum_f32(s, red) / (float)cols;
    float s2 = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const float d = Io<T>::get(xr + c) - mean;
        s2 += d * d;
    }
    const float rstd = 1.0f / sqrtf(block_sum_f32(s2, red) / (float)cols + eps);
    for (int64_t c = threadIdx.x; c < cols; c += blockDim.x) {
        const float d = Io<T>::get(xr + c) - mean;
        Io<T>::put(yr + c, add_rn(mul_rn(mul_rn(d, rstd), scale[c] + addend), shift[c]));
    }
}

template <typename T, int VPL>
void launch_wave(const void* x, int64_t xs, const float* shift, const float* scale, void* y,
                 int64_t ys, int rows, int nvec, int64_t cols, float eps, float addend,
                 hipStream_t st) {
    // One wave per row, four rows per workgroup; LDS holds the block's copy
    // of (scale + addend, shift): 8 bytes per column.  FULL rows (every lane
    // owns exactly VPL vectors) carry no bounds branches.
    constexpr int WPB = 4;
    const int blocks = (rows + WPB - 1) / WPB;
    const size_t lds = (size_t)nvec * Io<T>::EPV * 2 * sizeof(float);
    if (nvec == VPL * kWave)
        hipLaunchKernelGGL((adaln_wave_kernel<T, VPL, true, WPB>), dim3(blocks), dim3(WPB * kWave), lds, st,
                           (const T*)x, xs, shift, scale, (T*)y, ys, rows, nvec, (float)cols, eps, addend);
    else
        hipLaunchKernelGGL((adaln_wave_kernel<T, VPL, false, WPB>), dim3(blocks), dim3(WPB * kWave), lds, st,
                           (const T*)x, xs, shift, scale, (T*)y, ys, rows, nvec, (float)cols, eps, addend);
}

template <typename T>
int run(const void* x, int64_t rows, int64_t cols, int64_t xs, const float* shift,
        const float* scale, float addend, void* y, int64_t ys, float eps, hipStream_t st) {
    constexpr int EPV = Io<T>::EPV;
    const int64_t nvec = cols / EPV;
    const bool vec_ok = cols % EPV == 0 && xs % EPV == 0 && ys % EPV == 0 && aligned16(x) &&
                        aligned16(y) && aligned16(shift) && aligned16(scale) &&
                        nvec <= 16 * kWave && rows < (1ll << 31);
    if (vec_ok) {
        const int vpl = (int)((nvec + kWave - 1) / kWave);
        const int r = (int)rows, nv = (int)nvec;
        if (vpl <= 1) launch_wave<T, 1>(x, xs, shift, scale, y, ys, r, nv, cols, eps, addend, st);
        else if (vpl <= 2) launch_wave<T, 2>(x, xs, shift, scale, y, ys, r, nv, cols, eps, addend, st);
        else if (vpl <= 4) launch_wave<T, 4>(x, xs, shift, scale, y, ys, r, nv, cols, eps, addend, st);
        else if (vpl <= 6) launch_wave<T, 6>(x, xs, shift, scale, y, ys, r, nv, cols, eps, addend, st);
        else if (vpl <= 8) launch_wave<T, 8>(x, xs, shift, scale, y, ys, r, nv, cols, eps, addend, st);
        else if (vpl <= 12) launch_wave<T, 12>(x, xs, shift, scale, y, ys, r, nv, cols, eps, addend, st);
        else launch_wave<T, 16>(x, xs, shift, scale, y, ys, r, nv, cols, eps, addend, st);
    } else {
        DT_REQUIRE(rows <= 0x7FFFFFFF, "dt_adaln_mod: too many rows for the generic path");
        hipLaunchKernelGGL((adaln_generic_kernel<T>), dim3((unsigned)rows), dim3(256), 0, st,
                           (const T*)x, xs, shift, scale, (T*)y, ys, cols, eps, addend);
    }
    return check_launch("dt_adaln_mod");
}

template <typename T, int VPL>
void launch_res(const void* h, int64_t hs, const void* o, int64_t os, const float* gate, void* r, int64_t rs,
                const float* shift, const float* scale, void* y, int64_t ys, int rows, int nvec, int64_t cols,
                float eps, float addend, hipStream_t st) {
    // Six rows per workgroup: with (gate, 1 + scale, shift) in LDS, 12 bytes
    // per column, four workgroups of six rows fit a CU at 3072 columns.
    constexpr int WPB = 6;
    const int blocks = (rows + WPB - 1) / WPB;
    const size_t lds = (size_t)nvec * Io<T>::EPV * 3 * sizeof(float);
    if (nvec == VPL * kWave)
        hipLaunchKernelGGL((residual_adaln_kernel<T, VPL, true, WPB>), dim3(blocks), dim3(WPB * kWave), lds, st,
                           (const T*)h, hs, (const T*)o, os, gate, (T*)r, rs, shift, scale, (T*)y, ys, rows, nvec,
                           (float)cols, eps, addend);
    else
        hipLaunchKernelGGL((residual_adaln_kernel<T, VPL, false, WPB>), dim3(blocks), dim3(WPB * kWave), lds, st,
                           (const T*)h, hs, (const T*)o, os, gate, (T*)r, rs, shift, scale, (T*)y, ys, rows, nvec,
                           (float)cols, eps, addend);
}

template <typename T>
int run_res(const void* h, int64_t hs, const void* o, int64_t os, const float* gate, void* r, int64_t rs,
            const float* shift, const float* scale, float addend, void* y, int64_t ys, int64_t rows, int64_t cols,
            float eps, hipStream_t st) {
    constexpr int EPV = Io<T>::EPV;
    const int64_t nvec = cols / EPV;
    const bool fused = cols % EPV == 0 && hs % EPV == 0 && os % EPV == 0 && rs % EPV == 0 && ys % EPV == 0 &&
                       aligned16(h) && aligned16(o) && aligned16(r) && aligned16(y) && aligned16(gate) &&
                       aligned16(shift) && aligned16(scale) && nvec <= 16 * kWave && rows < (1ll << 31);
    if (!fused) {
        // rows the one-pass kernel does not take: the two launches it replaces
        const int rc = dt_gated_residual(h, hs, o, os, gate, r, rs, rows, cols, Io<T>::kType, st);
        if (rc) return rc;
        return adaln_launch(r, rows, cols, rs, shift, scale, addend, y, ys, eps, Io<T>::kType, st);
    }
    const int vpl = (int)((nvec + kWave - 1) / kWave);
    const int rw = (int)rows, nv = (int)nvec;
    if (vpl <= 2) launch_res<T, 2>(h, hs, o, os, gate, r, rs, shift, scale, y, ys, rw, nv, cols, eps, addend, st);
    else if (vpl <= 4) launch_res<T, 4>(h, hs, o, os, gate, r, rs, shift, scale, y, ys, rw, nv, cols, eps, addend, st);
    else if (vpl <= 6) launch_res<T, 6>(h, hs, o, os, gate, r, rs, shift, scale, y, ys, rw, nv, cols, eps, addend, st);
    else if (vpl <= 8) launch_res<T, 8>(h, hs, o, os, gate, r, rs, shift, scale, y, ys, rw, nv, cols, eps, addend, st);
    else if (vpl <= 12)
        launch_res<T, 12>(h, hs, o, os, gate, r, rs, shift, scale, y, ys, rw, nv, cols, eps, addend, st);
    else launch_res<T, 16>(h, hs, o, os, gate, r, rs, shift, scale, y, ys, rw, nv, cols, eps, addend, st);
    return check_launch("dt_gated_residual_adaln");
}

}  // namespace

int residual_adaln_launch(const void* h, int64_t hs, const void* o, int64_t os, const float* gate, void* r,
                          int64_t rs, const float* shift, const float* scale, float addend, void* y, int64_t ys,
                          int64_t rows, int64_t cols, float eps, int32_t io, hipStream_t st) {
    DT_REQUIRE(rows >= 0 && cols > 0, "dt_gated_residual_adaln: bad shape rows=%lld cols=%lld", (long long)rows,
               (long long)cols);
    DT_REQUIRE(hs >= cols && os >= cols && rs >= cols && ys >= cols,
               "dt_gated_residual_adaln: stride smaller than cols");
    DT_REQUIRE(is_io_type(io), "dt_gated_residual_adaln: io_type %d unsupported", io);
    if (rows == 0) return DT_OK;
    DT_REQUIRE(h && o && gate && r && shift && scale && y, "dt_gated_residual_adaln: null pointer");
    if (io == DT_TYPE_F32)
        return run_res<float>(h, hs, o, os, gate, r, rs, shift, scale, addend, y, ys, rows, cols, eps, st);
    return run_res<bf16>(h, hs, o, os, gate, r, rs, shift, scale, addend, y, ys, rows, cols, eps, st);
}

int adaln_launch(const void* x, int64_t rows, int64_t cols, int64_t xs, const float* shift,
                 const float* scale, float addend, void* y, int64_t ys, float eps, int32_t io,
                 hipStream_t st) {
    DT_REQUIRE(rows >= 0 && cols > 0, "dt_adaln_mod: bad shape rows=%lld cols=%lld",
               (long long)rows, (long long)cols);
    DT_REQUIRE(xs >= cols && ys >= cols, "dt_adaln_mod: stride smaller than cols");
    DT_REQUIRE(is_io_type(io), "dt_adaln_mod: io_type %d unsupported", io);
    if (rows == 0) return DT_OK;
    DT_REQUIRE(x && y && shift && scale, "dt_adaln_mod: null pointer");
    if (io == DT_TYPE_F32) return run<float>(x, rows, cols, xs, shift, scale, addend, y, ys, eps, st);
    return run<bf16>(x, rows, cols, xs, shift, scale, addend, y, ys, eps, st);
}

}  // namespace dit

extern "C" int dt_gated_residual_adaln(const void* h, int64_t h_stride, const void* o, int64_t o_stride,
                                       const float* gate, void* r, int64_t r_stride, const float* shift,
                                       const float* scale, void* y, int64_t y_stride, int64_t rows, int64_t cols,
                                       float eps, int32_t io_type, dt_stream_t stream) {
    return dit::residual_adaln_launch(h, h_stride, o, o_stride, gate, r, r_stride, shift, scale, 1.0f, y, y_stride,
                                      rows, cols, eps, io_type, (hipStream_t)stream);
}

extern "C" int dt_adaln_mod(const void* x, int64_t rows, int64_t cols, int64_t x_stride,
                            const float* shift, const float* scale, void* y, int64_t y_stride,
                            float eps, int32_t io_type, dt_stream_t stream) {
    return dit::adaln_launch(x, rows, cols, x_stride, shift, scale, 1.0f, y, y_stride, eps, io_type,
                             (hipStream_t)stream);
}
