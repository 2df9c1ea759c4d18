// kernels.hpp -- internal launchers shared by the C-ABI entry points and the
// graph executor (graph.cpp).  Not part of the public ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "dit_hip.h"

struct dt_backend;

namespace dit {

// y = (x - mean) * rstd * (scale + addend) + shift per row.  The public
// dt_adaln_mod uses addend 1 (the reference's `1 + scale`); the graph
// executor passes addend 0 with an already-computed factor tensor.
int adaln_launch(const void* x, int64_t rows, int64_t cols, int64_t xs, const float* shift,
                 const float* scale, float addend, void* y, int64_t ys, float eps, int32_t io,
                 hipStream_t st);

// r = h + gate * o; y = (r - mean) * rstd * (scale + addend) + shift per row,
// with r rounded to the I/O type before it is normalised.
int residual_adaln_launch(const void* h, int64_t hs, const void* o, int64_t os, const float* gate, void* r,
                          int64_t rs, const float* shift, const float* scale, float addend, void* y, int64_t ys,
                          int64_t rows, int64_t cols, float eps, int32_t io, hipStream_t st);

constexpr int kMaxRopeAxes = 8;

// Position of token t on axis a: ptr[a][t * stride[a]].
struct RopeAxisPos {
    const int32_t* ptr[kMaxRopeAxes];
    int64_t stride[kMaxRopeAxes];
};

int qk_launch(const void* q, const void* k, void* q_out, void* k_out, const float* wq,
              const float* wk, int64_t tokens, int64_t heads, int64_t head_dim, int64_t in_ts,
              int64_t in_hs, int64_t out_ts, int64_t out_hs, float eps, const RopeAxisPos& pos,
              int n_axes, int axis_dim, float freq_base, const float* table, int n_pos, int32_t io,
              hipStream_t st);

// The (cos, sin) table of dt_rope_table_fill's layout, [n_pos][axis_dim],
// computed on the device by the same recurrence the QK kernels use when they
// have no table: a kernel reading it gets the same bits as one computing the
// angles itself.  axis_dim % 8 == 0.
int rope_table_device(float* table, int n_pos, int axis_dim, float freq_base, hipStream_t st);

// Attention whose q is taken before its QK-RMSNorm + RoPE (dt_flash_attn_qk_bf16):
// q segment i covers queries [0, split) (i = 0) or [split, seq_q) (i = 1,
// token - split), with strides qs[i] = {batch, token, head} and norm
// weights w[i]; pos holds the joint sequence's positions per axis.
struct AttnQk {
    const void* q[2];
    int64_t qs[2][3];
    const float* w[2];
    int64_t split;
    float eps;
    RopeAxisPos pos;
    int n_axes, axis_dim;
    float freq_base;
    const float* table;
    int n_pos;
};
int flash_attn_qk_launch(const AttnQk& qk, const void* k, const void* v, void* o, int64_t batch, int64_t heads,
                         int64_t seq_q, int64_t seq_kv, const int64_t* k_strides, const int64_t* v_strides,
                         const int64_t* o_strides, float scale, int32_t o_type, hipStream_t st);

// QK-RMSNorm+RoPE of q and k (qk_launch's arguments) and a SwiGLU over
// gate/up rows -> y, in one launch when both take their fast paths.
int qk_swiglu_launch(const void* q, const void* k, void* q_out, void* k_out, const float* wq, const float* wk,
                     int64_t tokens, int64_t heads, int64_t head_dim, int64_t in_ts, int64_t in_hs, int64_t out_ts,
                     int64_t out_hs, float eps, const RopeAxisPos& pos, int n_axes, int axis_dim, float freq_base,
                     const float* table, int n_pos, const void* g, int64_t gs, const void* u, int64_t us, void* y,
                     int64_t ys, int64_t rows, int64_t cols, int32_t io, hipStream_t st);

// GroupNorm statistics written by the conv epilogue (dt_conv2d_gn): a head
// of N * G (mean, variance) double2, padded to 256 bytes, then the per-tile
// (mean, M2, count, 0) float4 records [N][G][pixel tiles].  The finalize step
// (groupnorm.hip) merges the records into the head.
inline int64_t gn_tile_stats_head_bytes(int64_t N, int64_t G) { return (N * G * 16 + 255) / 256 * 256; }
int gn_tile_stats_finalize(const void* stats, int64_t N, int64_t groups, int64_t n_tiles, hipStream_t st);
// The current device's address of dt_groupnorm_silu_noalloc's scratch array
// (resolved once per device).
int noalloc_scratch(void** out);

// Backend accessors (capi.cpp).
hipStream_t backend_stream(dt_backend* be);
int backend_device(dt_backend* be);
// Backend-owned scratch of at least `bytes` (grown on demand, freed with the backend).
int backend_scratch(dt_backend* be, size_t bytes, void** out);

// The backend's RoPE (cos, sin) table for positions [0, kBackendRopePositions)
// of one axis_dim / freq_base (rope_table_device; rebuilt when they change).
constexpr int kBackendRopePositions = 4096;
int backend_rope_table(dt_backend* be, int axis_dim, float freq_base, const float** out);

// Whether dt_conv2d with a workspace runs a K x K conv on io_type through
// the channel-last copy and the DMA kernel (else the register-staged kernel).
inline bool conv_uses_dma(int64_t K, int32_t io_type) { return K == 3 || (K == 1 && io_type == DT_TYPE_BF16); }

// Work the graph executor folds into a dt_conv2d (+ bias) launch
// (conv2d.hip: conv2d_fold).
struct ConvFold {
    // GroupNorm (+ affine) (+ SiLU) of the conv's input, applied as the 3x3
    // conv's channel-last copy reads it: (mean, rstd) per (n, group) from
    // gn_mean_rstd, the per-channel weight and bias (or null), the SiLU flag.
    // The copy stores the values the unfused GroupNorm would (then rounded
    // to bf16 as the copy rounds any input).
    const float2* gn_mr = nullptr;
    const float* gn_w = nullptr;
    const float* gn_b = nullptr;
    int gn_groups = 0;
    int gn_silu = 0;
    // ResnetBlock2D's residual: y = res + conv (res_mode 1) or (res + conv) *
    // res_scale (2), the conv output, the sum and the product each rounded
    // to the I/O type as the unfused nodes store them.  res has the output's
    // shape and type; it may be y itself (each element is read by the thread
    // that then writes it) but must not overlap y otherwise.
    const void* res = nullptr;
    int res_mode = 0;
    float res_scale = 1.0f;
};
// dt_conv2d with `fold`; y must not overlap the conv's input x (read around
// each output pixel).  The GroupNorm fold needs a 3x3 conv and a workspace.
int conv2d_fold(const void* x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void* packed_w, int64_t Co,
                int64_t K, int32_t upscale2, const float* bias, const ConvFold& fold, void* y, void* workspace,
                size_t workspace_bytes, int32_t io_type, hipStream_t st);

// GroupNorm statistics of x (NCHW, groups of C / groups channels) as
// (mean, rstd) per (n, group) in mr[N * groups], with exactly the values
// the two-pass dt_groupnorm_silu applies (groupnorm.hip); workspace as
// dt_groupnorm_silu's (dt_groupnorm_workspace_bytes).
int gn_mean_rstd(const void* x, int64_t N, int64_t C, int64_t HW, int64_t groups, float eps, void* workspace,
                 float2* mr, int32_t io_type, hipStream_t st);

}  // namespace dit
