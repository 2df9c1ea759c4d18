/*
 * dit_hip.h -- C ABI of libdit_hip.so: MI355X (gfx950) kernels for the
 * Flux2 DiT elementwise / reduction / broadcast chain of diffusers-cpp.
 *
 * The reference reaches this arithmetic through its `Runtime` op-builder
 * (src/ggml/Runtime.hpp:7-317), which forwards 1:1 to ggml
 * (src/ggml/ExecutionRuntime.cpp:319-766) and executes the graph with
 * ggml_backend_graph_compute (src/ggml/ExecutionRuntime.cpp:227, 254).
 * This library replaces the ggml backend for that op subset.  It exposes
 * three groups of entry points:
 *
 *   (i)   a ggml-shaped tensor descriptor and graph executor (dt_graph_*),
 *         which pattern-matches the op chains the reference emits and
 *         lowers them to the fused kernels;
 *   (ii)  the fused kernels themselves (dt_adaln_mod, dt_qk_rmsnorm_rope,
 *         dt_swiglu, dt_gated_residual, dt_dequant, dt_groupnorm_silu);
 *   (iii) unfused single-op kernels with ggml semantics (dt_op_*), used
 *         where no fusion pattern applies.
 *
 * Conventions
 *  - Every pointer named x/y/src/dst/... is DEVICE memory owned by the
 *    caller; the library allocates device memory only in dt_buffer_alloc
 *    and for a dt_backend's own state, made by its first dt_graph_compute
 *    that needs it (scratch and RoPE table)
 *    and freed by dt_backend_free.
 *  - `stream` is a hipStream_t (NULL = the default stream).  All kernels are
 *    stream-ordered and asynchronous; none synchronises the device.
 *  - Strides are in ELEMENTS unless named *_bytes / nb.
 *  - Every function returns 0 (DT_OK) or a DT_ERR_* code and never aborts;
 *    dt_last_error() returns a thread-local message for the last failure.
 *  - Threads: the kernel entry points ((ii), (iii)) keep no state and may be
 *    called from any thread.  A dt_backend (its scratch and RoPE table)
 *    and the nodes given to its dt_graph_* calls are used
 *    by one host thread at a time, as the reference builds and computes a
 *    graph on the thread whose Scope holds it (thread_local,
 *    src/ggml/Scope.hpp:74-75); separate backends may run on separate
 *    threads.
 *  - io_type selects the element type of activations: DT_TYPE_F32 or
 *    DT_TYPE_BF16 (all arithmetic is fp32 either way).  Modulation vectors,
 *    norm weights and rope tables are always fp32.
 */
#ifndef DIT_HIP_H
#define DIT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* ggml type ids (ggml.h enum ggml_type), kept numerically identical, plus
 * two backend weight layouts made once at load (no ggml counterpart; ggml
 * likewise repacks weights into backend layouts through its "extra" buffer
 * types):
 * DT_TYPE_Q8_0_SPLIT: a Q8_0 Linear weight [N][K] repacked by dt_q8_0_split
 * for dt_gemm_q8_0.  A tensor of this type has ne = {K, N, 1, 1}, nb = {1, K,
 * N K, N K}; its data holds the uint8 codes [N][K] at offset 0 and the fp32
 * block scales [K/32][N] at dt_q8_0_split_scale_offset(N, K).
 * DT_TYPE_CONV2D_PACKED: a Conv2d weight [Co][Ci][K][K] packed by
 * dt_conv2d_pack_weights, the layout dt_conv2d reads (ne = {K, K, Ci, Co},
 * dt_conv2d_packed_bytes(Co, Ci, K) bytes; nb is not used).  As src0 of
 * DT_OP_CONV_2D_DIRECT it spares the executor a repack per call. */
enum {
    DT_TYPE_F32 = 0,
    DT_TYPE_F16 = 1,
    DT_TYPE_Q8_0 = 8,
    DT_TYPE_Q4_K = 12,
    DT_TYPE_I32 = 26,
    DT_TYPE_BF16 = 30,
    DT_TYPE_Q8_0_SPLIT = 100,
    DT_TYPE_CONV2D_PACKED = 101
};

enum {
    DT_OK = 0,
    DT_ERR_INVALID_ARG = 1,
    DT_ERR_UNSUPPORTED = 2,
    DT_ERR_HIP = 3,
    DT_ERR_OOM = 4
};

typedef void *dt_stream_t; /* hipStream_t */

const char *dt_last_error(void);
const char *dt_version(void);

/* ======================================================================== */
/* (ii) fused entry points                                                  */
/* ======================================================================== */

/* adaLN: y = (1 + scale) * LayerNorm_eps(x) + shift, per row of `cols`.
 * Replaces the NORM -> ADD(scale,1) -> MUL -> ADD node chain emitted by
 * LayerNorm::forward (src/nn/modules/normalization/LayerNorm.cpp:16-32,
 * Runtime::norm at src/ggml/Runtime.hpp:273-275) followed by the modulation
 * in Flux2SingleTransformerBlock.hpp:50-54, Flux2TransformerBlock.hpp:63-72,
 * 91-92, 105-106 and AdaLayerNormContinuous.inl:38-40.
 * shift/scale: fp32 [cols] (the chunk views of the Flux2Modulation output). */
int dt_adaln_mod(const void *x, int64_t rows, int64_t cols, int64_t x_stride,
                 const float *shift, const float *scale,
                 void *y, int64_t y_stride, float eps, int32_t io_type,
                 dt_stream_t stream);

/* QK-RMSNorm + multi-axis RoPE for q and k in one launch:
 *   z = RMSNorm_eps(x[t,h,:]) * w ;  y[t,h,:] = cat_a RoPE_NORMAL(z[a-th section], pos[t,a])
 * Replaces RMSNorm::forward (src/nn/modules/normalization/RMSNorm.cpp:12-22,
 * Runtime::rms_norm at src/ggml/Runtime.hpp:277-279) on the unflattened q/k
 * (Flux2Attention.hpp:93-112, Flux2ParallelSelfAttention.hpp:63-76) and
 * Flux2PosEmbed::forward (Flux2PosEmbed.hpp:18-109: four Runtime::rope_ext,
 * src/ggml/Runtime.hpp:281-293, mode NORMAL, plus Tensor::cat).
 * Layout: element (t, h, d) of q/k at t*tok_stride + h*head_stride + d.
 * q or k may be NULL (that half is skipped); q_out may alias q.
 * pos: int32, position of token t on axis a at pos[t*pos_stride + a].
 * n_axes * axis_dim must equal head_dim.  rope_table: fp32
 * [n_pos][axis_dim] holding (cos, sin) pairs as filled by
 * dt_rope_table_fill for the same axis_dim/freq_base (NULL or n_pos = 0:
 * angles are computed on the device); positions outside [0, n_pos) are
 * computed on the device. */
int dt_qk_rmsnorm_rope(const void *q, const void *k, void *q_out, void *k_out,
                       int64_t tokens, int64_t heads, int64_t head_dim,
                       int64_t in_tok_stride, int64_t in_head_stride,
                       int64_t out_tok_stride, int64_t out_head_stride,
                       const float *wq, const float *wk, float eps,
                       const int32_t *pos, int64_t pos_stride,
                       int32_t n_axes, int32_t axis_dim, float freq_base,
                       const float *rope_table, int32_t n_pos,
                       int32_t io_type, dt_stream_t stream);

/* Host-side: fill table[p*n_dims + 2i] = cos(theta_i(p)) * attn_factor and
 * table[p*n_dims + 2i + 1] = sin(...) for p < n_pos, i < n_dims/2, with
 * ggml's fp32 angle recurrence theta_0 = p*freq_scale,
 * theta_{i+1} = theta_i * powf(freq_base, -2/n_dims) (the rope cache of
 * ggml_rope_ext with ext_factor 0).  `table` is HOST memory of
 * n_pos*n_dims floats; upload it once per model. */
int dt_rope_table_fill(float *table, int32_t n_pos, int32_t n_dims,
                       float freq_base, float freq_scale, float attn_factor);

/* SwiGLU: y = silu(gate) * up = (gate * sigmoid(gate)) * up.
 * Replaces SIGMOID -> MUL -> MUL of Flux2SwiGLU::forward
 * (Flux2SwiGLU.hpp:17-21, SiLU.hpp:9-13; Runtime::sigmoid/mul at
 * src/ggml/Runtime.hpp:89-91, 107-110). Rows of `inner` elements. */
int dt_swiglu(const void *gate, int64_t gate_stride, const void *up, int64_t up_stride,
              void *y, int64_t y_stride, int64_t rows, int64_t inner,
              int32_t io_type, dt_stream_t stream);

/* Gated residual: y = h + gate * o, gate fp32 [cols] broadcast over rows.
 * Replaces MUL -> ADD of Flux2SingleTransformerBlock.hpp:58 and
 * Flux2TransformerBlock.hpp:86-87, 97, 100-101, 111.  y may alias h. */
int dt_gated_residual(const void *h, int64_t h_stride, const void *o, int64_t o_stride,
                      const float *gate, void *y, int64_t y_stride,
                      int64_t rows, int64_t cols, int32_t io_type, dt_stream_t stream);

/* dt_qk_rmsnorm_rope (q and k) and dt_swiglu in one launch: the three
 * elementwise ops a Flux2 single-stream block applies to the outputs of its
 * input projections (Flux2ParallelSelfAttention.hpp:55-93), which are all
 * ready at once.  Arguments are those of the two functions (q or k may be
 * NULL: with the block's q taken by dt_flash_attn_qk_bf16, k and the SwiGLU
 * still share one launch); results are bit-identical to calling them
 * separately (which is what happens for shapes the combined kernel does not
 * take). */
int dt_qk_rmsnorm_rope_swiglu(const void *q, const void *k, void *q_out, void *k_out, int64_t tokens,
                              int64_t heads, int64_t head_dim, int64_t in_tok_stride,
                              int64_t in_head_stride, int64_t out_tok_stride, int64_t out_head_stride,
                              const float *wq, const float *wk, float eps, const int32_t *pos,
                              int64_t pos_stride, int32_t n_axes, int32_t axis_dim, float freq_base,
                              const float *rope_table, int32_t n_pos, const void *gate,
                              int64_t gate_stride, const void *up, int64_t up_stride, void *y,
                              int64_t y_stride, int64_t rows, int64_t inner, int32_t io_type,
                              dt_stream_t stream);

/* Gated residual and the next adaLN in one pass (fused across a block
 * boundary): r = h + gate * o (Flux2SingleTransformerBlock.hpp:58,
 * Flux2TransformerBlock.hpp:86-87, 100-101), then y = (1 + scale) *
 * LayerNorm_eps(r) + shift (the next block's adaLN, Flux2SingleTransformerBlock.hpp:50-54,
 * Flux2TransformerBlock.hpp:63-72, 91-92).  r is written, rounded to io_type,
 * and that rounded value is what is normalised, as in the unfused graph.
 * gate, shift, scale: fp32 [cols].  Rows 16-byte aligned, cols % 8 == 0
 * (bf16) or % 4 (fp32), cols <= 4096 (bf16) / 2048 (fp32). */
int dt_gated_residual_adaln(const void *h, int64_t h_stride, const void *o, int64_t o_stride,
                            const float *gate, void *r, int64_t r_stride, const float *shift,
                            const float *scale, void *y, int64_t y_stride, int64_t rows, int64_t cols,
                            float eps, int32_t io_type, dt_stream_t stream);

/* Weight dequantisation to dst_type (DT_TYPE_BF16 or DT_TYPE_F32).
 * qtype DT_TYPE_Q8_0 (cols % 32 == 0) or DT_TYPE_Q4_K (cols % 256 == 0);
 * ggml blocks run along cols (ne0); row r starts at src + r*row_bytes.
 * fp32 value = d*q (Q8_0) or (d*sc)*q - (dmin*m) (Q4_K), each operation
 * rounded; bf16 output is the RNE rounding of that value.  Stands in for the
 * implicit dequantisation inside Runtime::mul_mat (src/ggml/Runtime.hpp:136-139)
 * of Linear::forward (src/nn/Linear.cpp:17-36) on Q8_0/Q4_K GGUF weights. */
int dt_dequant(const void *src, int32_t qtype, int64_t rows, int64_t cols,
               int64_t row_bytes, void *dst, int64_t dst_stride, int32_t dst_type,
               dt_stream_t stream);

/* GroupNorm(groups, eps) over x[N][C][HW] (NCHW, contiguous), optional
 * per-channel affine (w, b may be NULL), then SiLU when apply_silu.
 * Replaces GroupNorm::forward (src/nn/modules/normalization/GroupNorm.cpp:25-108:
 * reshape -> NORM -> reshape -> MUL -> ADD) and SiLU::forward
 * (SiLU.hpp:9-13) as used in ResnetBlock2D.inl:111-122, 160-171 and
 * Decoder.hpp:147-160.  `workspace` is caller-owned device memory of at
 * least dt_groupnorm_workspace_bytes(...) bytes.  y may alias x.  An empty
 * input (N == 0 or HW == 0) is a no-op that touches no pointer. */
size_t dt_groupnorm_workspace_bytes(int64_t N, int64_t C, int64_t HW, int64_t groups);
int dt_groupnorm_silu(const void *x, int64_t N, int64_t C, int64_t HW, int64_t groups,
                      const float *w, const float *b, float eps, int32_t apply_silu,
                      void *y, void *workspace, size_t workspace_bytes,
                      int32_t io_type, dt_stream_t stream);

/* dt_groupnorm_silu without a workspace argument and without allocating:
 * no counterpart in the reference.  For callers that cannot allocate device
 * memory (code under HIP graph capture, tight serving loops, harnesses that
 * forbid hipMalloc).  The statistics live in a device array of
 * DT_GROUPNORM_NOALLOC_SCRATCH_BYTES the library holds on every device it
 * runs on until the process ends; maps needing more statistics space (the
 * bytes dt_groupnorm_workspace_bytes would give for the vector path, e.g.
 * fp32 [1, 256, 1024, 1024] needs 1.05 MB) return DT_ERR_INVALID_ARG.  All
 * calls on one device share that array: calls that overlap on one device
 * (concurrent streams) race.  Same results as dt_groupnorm_silu, bit for
 * bit. */
#define DT_GROUPNORM_NOALLOC_SCRATCH_BYTES (2u << 20)
int dt_groupnorm_silu_noalloc(const void *x, int64_t N, int64_t C, int64_t HW, int64_t groups,
                              const float *w, const float *b, float eps, int32_t apply_silu, void *y,
                              int32_t io_type, dt_stream_t stream);

/* Euler step of FlowMatchEulerDiscreteScheduler::integrate
 * (src/diffusers/schedulers/FlowMatchEulerDiscreteScheduler.cpp:210-222):
 * y = x + dt * v over n contiguous elements. */
int dt_euler_step(const void *x, const void *v, float dt, void *y, int64_t n,
                  int32_t io_type, dt_stream_t stream);

/* Q8_0 blocks (rows x cols/32 blocks of {fp16 d; int8 qs[32]}, row_bytes
 * apart) -> the split layout dt_gemm_q8_0 reads: codes[r][c] = qs + 128 as
 * uint8 ([rows][ld_codes], ld_codes % 16 == 0) and scales[c / 32][r] = d as
 * fp32 ([cols/32][ld_scales]).  A one-time weight repack (the reference reads
 * the blocks from GGUF, src/ggml/GGUFLoaderVisitor.cpp:214-281). */
int dt_q8_0_split(const void *src, int64_t rows, int64_t cols, int64_t row_bytes, void *codes,
                  int64_t ld_codes, float *scales, int64_t ld_scales, dt_stream_t stream);
/* Layout of a DT_TYPE_Q8_0_SPLIT weight of `rows` x `cols`: byte offset of
 * its scales (the codes rounded up to 256 bytes) and its total size. */
int64_t dt_q8_0_split_scale_offset(int64_t rows, int64_t cols);
int64_t dt_q8_0_split_bytes(int64_t rows, int64_t cols);

/* Q8_0 quantisation of fp32 rows (ggml quantize_row_q8_0_ref semantics:
 * d = amax/127, q = roundf(x / d), d stored as RNE fp16).  cols % 32 == 0;
 * dst row r starts at dst + r*row_bytes.  Makes Q8_0 weight bytes on the
 * device, in place of the GGUF reader of src/ggml/GGUFLoaderVisitor.cpp:214-281. */
int dt_quantize_q8_0(const float *src, int64_t rows, int64_t cols, int64_t src_stride,
                     void *dst, int64_t row_bytes, dt_stream_t stream);

/* ---- VAE decoder convolutions ------------------------------------------------ */

/* Conv2d::forward (src/nn/modules/conv/Conv2d.cpp:37-108): ggml_conv_2d_direct
 * with stride 1, dilation 1, a square kernel K in {1, 3} and padding
 * (K - 1) / 2, then + bias[co]; NCHW, x [N][Ci][H][W] of io_type, y
 * [N][Co][H'][W'] of io_type.  With upscale2 the conv reads the nearest 2x
 * upscale of x (H' = 2H, W' = 2W), the `upscale(x, 2, NEAREST)` of
 * Upsample2D::forward (src/diffusers/models/resnet/Upsample2D.cpp:36-63),
 * which is then never stored.  Operands are rounded to bf16 (as in
 * dt_gemm_bf16), sums are fp32.  The weights must first be packed by
 * dt_conv2d_pack_weights into a buffer of dt_conv2d_packed_bytes. */
size_t dt_conv2d_packed_bytes(int64_t Co, int64_t Ci, int64_t K);
int dt_conv2d_pack_weights(const void *w, int32_t w_type, int64_t Co, int64_t Ci, int64_t K,
                           void *packed, dt_stream_t stream);
/* The caller's workspace of dt_conv2d_workspace_bytes (16-byte aligned)
 * holds a bf16 channel-last copy of x, from which both operands stream into
 * LDS by direct DMA; workspace NULL selects a slower path that stages x from
 * NCHW itself (same results). */
size_t dt_conv2d_workspace_bytes(int64_t N, int64_t Ci, int64_t H, int64_t W);
int dt_conv2d(const void *x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void *packed_w,
              int64_t Co, int64_t K, int32_t upscale2, const float *bias, void *y, void *workspace,
              size_t workspace_bytes, int32_t io_type, dt_stream_t stream);

/* dt_conv2d whose epilogue also reduces GroupNorm(groups) statistics of the
 * output it stores: per output tile and group a (mean, M2, count) record,
 * merged at the end into a head of N * groups (mean, variance) double pairs
 * at the start of `stats` (dt_conv2d_gn_stats_bytes; 16-byte aligned).  The
 * GroupNorm + SiLU that follows (ResnetBlock2D.inl:111-122, 160-171;
 * Decoder.hpp:147-160) is then one read and one write of the tensor,
 * dt_groupnorm_silu_from_stats, instead of dt_groupnorm_silu's statistics
 * pass plus apply pass.  Co / groups must divide 128.  The statistics are
 * merged in a fixed order (Chan's pairwise update, fp64): deterministic. */
size_t dt_conv2d_gn_stats_bytes(int64_t N, int64_t Co, int64_t OH, int64_t OW, int64_t groups);
int dt_conv2d_gn(const void *x, int64_t N, int64_t Ci, int64_t H, int64_t W, const void *packed_w,
                 int64_t Co, int64_t K, int32_t upscale2, const float *bias, void *y, int64_t groups,
                 void *stats, size_t stats_bytes, void *workspace, size_t workspace_bytes,
                 int32_t io_type, dt_stream_t stream);
/* GroupNorm(groups) + affine + optional SiLU of x with the statistics
 * dt_conv2d_gn wrote for it: y = silu(((x - mean) * rstd) * w_c + b_c),
 * rstd = 1 / sqrt(var + eps), as dt_groupnorm_silu applies them. */
int dt_groupnorm_silu_from_stats(const void *x, int64_t N, int64_t C, int64_t HW, int64_t groups,
                                 const void *stats, const float *w, const float *b, float eps,
                                 int32_t apply_silu, void *y, int32_t io_type, dt_stream_t stream);

/* ggml_upscale(x, factor, GGML_SCALE_MODE_NEAREST) of a contiguous NCHW
 * tensor: dst[n][c][i][j] = src[n][c][i / factor][j / factor]
 * (Upsample2D::forward, Upsample2D.cpp:36-63, when no conv consumes it). */
int dt_op_upscale_nearest(const void *src, int64_t N, int64_t C, int64_t H, int64_t W, int32_t factor, void *dst,
                          int32_t io_type, dt_stream_t stream);

/* Synthetic N(mean, std^2) fp32 data on the device (benchmark weights and
 * inputs; a seeded splitmix64 + Box-Muller stream).  No counterpart in the
 * reference, which reads weights from GGUF files. */
int dt_fill_randn(float *y, int64_t n, uint64_t seed, float mean, float std,
                  dt_stream_t stream);

/* ---- step-time support: Linear and attention ---------------------------- */

/* C[m][n] = sum_k A[m][k] * B[n][k] (+ bias[n]) (+ addend[m][n]), bf16 A and
 * B, fp32 accumulation, C of c_type (DT_TYPE_BF16 or DT_TYPE_F32; addend has
 * C's type and leading dimension ldd).  A is the activation [M, K] and B a
 * Linear weight [N, K] (PyTorch [out, in]), both K-contiguous: this is
 * Runtime::mul_mat(w, x) (src/ggml/Runtime.hpp:136-139) as called by
 * Linear::forward (src/nn/Linear.cpp:17-36), and with `addend` the
 * `attn(x) + mlp(y)` sum of Flux2FusedAttentionOutput::forward
 * (src/diffusers/models/transformers/flux2/Flux2FusedAttentionOutput.hpp:31-36).
 * Any K >= 1 and leading dimensions (A, B 2-byte aligned); K % 64 == 0 with
 * lda, ldb % 8 == 0 and A, B 16-byte aligned runs the tiled kernels, any
 * other shape a masked 128 x 128 kernel.  C may alias addend. */
int dt_gemm_bf16(const void *A, int64_t lda, const void *B, int64_t ldb, void *C, int64_t ldc,
                 int64_t M, int64_t N, int64_t K, const float *bias, const void *addend,
                 int64_t ldd, int32_t c_type, dt_stream_t stream);
/* dt_gemm_bf16 with the weight B kept as Q8_0 (GGUF Q8_0 blocks repacked
 * once by dt_q8_0_split): each weight is dequantised in the GEMM's load path,
 * d * q rounded to bf16, so C equals dt_dequant to bf16 followed by
 * dt_gemm_bf16 bit for bit (finite scales).  The weight stays 1.125 bytes per
 * element in HBM.  Replaces the same Runtime::mul_mat call as dt_gemm_bf16
 * for the reference's Q8_0 Linear weights (src/nn/Linear.cpp:17-36;
 * flux2-klein-9b-q8.json), whose CPU path dequantises inside ggml's matmul.
 * K % 32 == 0 (whole Q8_0 blocks); scales 4-byte aligned with ld_scales >= N;
 * K % 64 == 0 with ld_codes % 16 == 0 runs the tiled kernel, K % 64 == 32 the
 * masked one. */
int dt_gemm_q8_0(const void *A, int64_t lda, const void *codes, int64_t ld_codes, const float *scales,
                 int64_t ld_scales, void *C, int64_t ldc, int64_t M, int64_t N, int64_t K,
                 const float *bias, const void *addend, int64_t ldd, int32_t c_type,
                 dt_stream_t stream);

/* dt_gemm_bf16 with an explicit tile configuration: 0 = 256x256 per
 * workgroup with direct global->LDS loads in four K = 32 stages, 1 = 128x128
 * with two workgroups per CU (bf16 or Q8_0 weights; Q8_0 dequantised as it
 * is staged), 2 = 256x256 with two K = 64 stages, 3 = Q8_0 weights at
 * 256x256 in eight waves (dequantised after the LDS read), 4 = the masked
 * any-shape kernel (bf16 or Q8_0 weights), 5 =
 * config 2 with buffer loads to LDS and its LDS reads and loads interleaved
 * into the MFMA stream, 6 = config 5 with 224-row tiles, 7 = config 5 with
 * Q8_0 weights dequantised as they are staged, 8 = config 5 in eight waves
 * of 128x64 (two per SIMD; the 256x256 kernel dt_gemm_bf16 picks), 9 =
 * config 7 in eight waves (the Q8_0 one); -1 picks by shape as dt_gemm_bf16
 * does (bf16: 8 or 1; Q8_0: 9 or 1).  Every configuration gives the same
 * bits.  For tuning and tests; no counterpart in the reference. */
int dt_gemm_bf16_config(const void *A, int64_t lda, const void *B, int64_t ldb, void *C,
                        int64_t ldc, int64_t M, int64_t N, int64_t K, const float *bias,
                        const void *addend, int64_t ldd, int32_t c_type, int32_t config,
                        dt_stream_t stream);

/* One GEMM of a group: the arguments of dt_gemm_bf16.  With b_scale set, B
 * is a Q8_0 weight in the split layout of dt_q8_0_split (uint8 codes, ldb in
 * bytes, a multiple of 16) and b_scale its fp32 block scales
 * [K/32][ld_scale] (ld_scale >= N, 4-byte aligned); every problem of a group
 * must then be Q8_0. */
typedef struct dt_gemm_problem {
    const void *A;
    int64_t lda;
    const void *B;
    int64_t ldb;
    void *C;
    int64_t ldc;
    const void *addend;
    int64_t ldd;
    const float *bias;
    int64_t M, N, K;
    const float *b_scale;
    int64_t ld_scale;
} dt_gemm_problem;

/* Up to 8 independent GEMMs (same c_type) in one launch whose tiles share
 * the grid, e.g. the q, k, v, gate and up projections Linear::forward issues
 * one after another on the same input (Flux2FusedQKVProjection.hpp:61-68,
 * Flux2Attention.hpp:64-83, Flux2FeedForward.hpp:62-72).  No outputs may
 * overlap another problem's inputs.  config as for dt_gemm_bf16_config. */
int dt_gemm_bf16_grouped(const dt_gemm_problem *problems, int32_t count, int32_t c_type,
                         int32_t config, dt_stream_t stream);

/* Unmasked attention softmax(scale * Q K^T) V per (batch, head), head_dim
 * 128, bf16 q/k/v, fp32 softmax and accumulation, o of o_type (BF16 or F32).
 * Element (b, s, h, d) of q is q[b*q_strides[0] + s*q_strides[1] +
 * h*q_strides[2] + d]; likewise k, v (seq_kv tokens) and o (seq_q tokens).
 * Replaces Runtime::flash_attn_ext (src/ggml/Runtime.hpp:250-257) as called
 * by FlashAttentionOp::operator() (src/nn/attention/FlashAttentionOp.cpp:84-94)
 * with no mask; strides are multiples of 8 (q, k, v) / 4 (o) elements. */
int dt_flash_attn_bf16(const void *q, const void *k, const void *v, void *o, int64_t batch,
                       int64_t heads, int64_t seq_q, int64_t seq_kv, int64_t head_dim,
                       const int64_t *q_strides, const int64_t *k_strides,
                       const int64_t *v_strides, const int64_t *o_strides, float scale,
                       int32_t o_type, dt_stream_t stream);

/* dt_flash_attn_bf16 with q taken BEFORE its QK-RMSNorm + RoPE: the kernel
 * applies dt_qk_rmsnorm_rope's transform (RMSNorm over the 128 dims with
 * eps and the fp32 weights, then the n_axes x axis_dim NORMAL-mode
 * rotations at the query's positions) to each query as it loads it, so the
 * normalised q is never stored and read back -- the q half of
 * Flux2Attention.hpp:93-122 / Flux2ParallelSelfAttention.hpp:63-76 folded
 * into FlashAttentionOp::operator() (FlashAttentionOp.cpp:84-94).
 * Queries [0, split) come from q0 (token t at q0 + b*q0_strides[0] +
 * t*q0_strides[1] + h*q0_strides[2], weights w0), queries [split, seq_q)
 * from q1 (token t - split, weights w1): the txt | img concatenation of the
 * double-stream attention; split >= seq_q leaves q1 / q1_strides / w1 unused.
 * pos, pos_stride, n_axes, axis_dim, freq_base, rope_table and n_pos are
 * dt_qk_rmsnorm_rope's (positions of the joint sequence; axis_dim % 8 == 0).
 * The result is bit-identical to dt_qk_rmsnorm_rope with the same table
 * followed by dt_flash_attn_bf16. */
int dt_flash_attn_qk_bf16(const void *q0, const int64_t *q0_strides, const float *w0,
                          const void *q1, const int64_t *q1_strides, const float *w1, int64_t split,
                          float eps, const int32_t *pos, int64_t pos_stride, int32_t n_axes,
                          int32_t axis_dim, float freq_base, const float *rope_table, int32_t n_pos,
                          const void *k, const void *v, void *o, int64_t batch, int64_t heads,
                          int64_t seq_q, int64_t seq_kv, int64_t head_dim, const int64_t *k_strides,
                          const int64_t *v_strides, const int64_t *o_strides, float scale,
                          int32_t o_type, dt_stream_t stream);

/* fp32 counterparts for graphs whose weights and activations are both F32
 * (the reference's own precision: Linear::forward with F32 weights,
 * src/nn/Linear.cpp:17-36, and FlashAttentionOp::operator() on F32 q/k/v,
 * src/nn/attention/FlashAttentionOp.cpp:84-94).  Products and sums in fp32
 * on the fp32 matrix cores.
 * dt_gemm_f32: C = A B^T (+ bias) (+ addend) as dt_gemm_bf16 with fp32 A
 * [M, K], B [N, K], C and addend (any K; A, B 4-byte aligned; with N % 4 == 0
 * C 16-byte aligned and ldc % 4 == 0).  dt_gemm_f32_grouped: up to 8 of them
 * in one launch (b_scale must be NULL).
 * dt_flash_attn_f32: softmax(scale Q K^T) V per (batch, head), strides as
 * dt_flash_attn_bf16, fp32 o; the scores of up to 8 heads at a time go
 * through `workspace` (dt_flash_attn_f32_workspace_bytes, 16-byte aligned). */
int dt_gemm_f32(const float *A, int64_t lda, const float *B, int64_t ldb, float *C, int64_t ldc, int64_t M,
                int64_t N, int64_t K, const float *bias, const float *addend, int64_t ldd, dt_stream_t stream);
int dt_gemm_f32_grouped(const dt_gemm_problem *problems, int32_t count, dt_stream_t stream);
size_t dt_flash_attn_f32_workspace_bytes(int64_t batch, int64_t heads, int64_t seq_q, int64_t seq_kv,
                                         int64_t head_dim);
int dt_flash_attn_f32(const float *q, const float *k, const float *v, float *o, int64_t batch, int64_t heads,
                      int64_t seq_q, int64_t seq_kv, int64_t head_dim, const int64_t *q_strides,
                      const int64_t *k_strides, const int64_t *v_strides, const int64_t *o_strides, float scale,
                      void *workspace, size_t workspace_bytes, dt_stream_t stream);

/* ======================================================================== */
/* (iii) unfused ggml-op kernels on ggml-shaped descriptors                 */
/* ======================================================================== */

/* A ggml_tensor-shaped descriptor: ne[] ggml order (ne[0] fastest),
 * nb[] byte strides, device data.  op/op_params/src describe graph nodes
 * for dt_graph_compute; single-op kernels read only type/ne/nb/data. */
typedef struct dt_tensor {
    int32_t type;
    int32_t op;
    int64_t ne[4];
    int64_t nb[4];
    void *data;
    int32_t op_params[16];
    struct dt_tensor *src[4];
    int32_t flags;
    int32_t id;
} dt_tensor;

/* Binary ops with ggml broadcast (src1 repeats into src0's shape, dst has
 * src0's shape): Runtime::add/sub/mul/div (src/ggml/Runtime.hpp:97-115). */
enum { DT_BIN_ADD = 0, DT_BIN_SUB = 1, DT_BIN_MUL = 2, DT_BIN_DIV = 3 };
int dt_op_binary(int32_t op, const dt_tensor *src0, const dt_tensor *src1,
                 const dt_tensor *dst, dt_stream_t stream);

/* Unary ops: Runtime::sigmoid/exp/log/sqrt/sin/cos (Runtime.hpp:69-91),
 * scale (:121-124, p0 = factor), clamp (:126-130, p0 = min, p1 = max),
 * SILU (x * sigmoid(x), the SiLU module's composite). */
enum {
    DT_UN_SIGMOID = 0, DT_UN_EXP = 1, DT_UN_LOG = 2, DT_UN_SQRT = 3,
    DT_UN_SIN = 4, DT_UN_COS = 5, DT_UN_SCALE = 6, DT_UN_CLAMP = 7,
    DT_UN_SILU = 8, DT_UN_FILL = 9
};
int dt_op_unary(int32_t op, const dt_tensor *src, const dt_tensor *dst,
                float p0, float p1, dt_stream_t stream);

/* Row norms over ne[0]: Runtime::norm / rms_norm (Runtime.hpp:273-279). */
int dt_op_norm(const dt_tensor *src, const dt_tensor *dst, float eps, dt_stream_t stream);
int dt_op_rms_norm(const dt_tensor *src, const dt_tensor *dst, float eps, dt_stream_t stream);

/* Runtime::rope_ext (Runtime.hpp:281-293), mode 0 (NORMAL) only, no
 * frequency factors, ext_factor 0.  pos: int32 [src->ne[2]] device. */
int dt_op_rope_ext(const dt_tensor *src, const int32_t *pos, const dt_tensor *dst,
                   int32_t n_dims, int32_t mode, float freq_base, float freq_scale,
                   float ext_factor, float attn_factor, dt_stream_t stream);

/* Runtime::concat (Runtime.hpp:236-240) along ggml dim `dim`; same-type
 * operands of any 2/4-byte type (I32 included) are copied bit for bit. */
int dt_op_concat(const dt_tensor *a, const dt_tensor *b, int32_t dim,
                 const dt_tensor *dst, dt_stream_t stream);

/* Runtime::cont / cpy / cast (Runtime.hpp:47-63): strided copy with
 * conversion between F32, F16 and BF16 (same element count); same-type
 * copies (I32 included) move the bits unchanged. */
int dt_op_cpy(const dt_tensor *src, const dt_tensor *dst, dt_stream_t stream);

/* ======================================================================== */
/* (i) device, buffers and graph execution                                  */
/* ======================================================================== */

typedef struct dt_backend dt_backend;

/* Device / Backend / Buffer RAII stand-ins (src/ggml/Device.hpp:8-27,
 * Backend.hpp:5-31, Buffer.hpp:8-42). */
int dt_backend_init(int32_t device_ordinal, dt_backend **out);
int dt_backend_free(dt_backend *be);
/* The caller's stream from now on.  A stream the backend created itself
 * (dt_graph_capture on the NULL stream) is synchronised and destroyed; the
 * caller's stream is never destroyed by the library. */
int dt_backend_set_stream(dt_backend *be, dt_stream_t stream);
int dt_backend_synchronize(dt_backend *be);
int dt_buffer_alloc(dt_backend *be, size_t bytes, void **out);
int dt_buffer_free(dt_backend *be, void *ptr);
/* ggml_backend_tensor_set / get: n bytes at byte offset of a contiguous
 * tensor; offset + n must lie within the tensor's bytes (DT_ERR_INVALID_ARG
 * otherwise, as ggml asserts offset + size <= ggml_nbytes). */
int dt_tensor_set(const dt_tensor *t, const void *host, size_t offset, size_t n, dt_stream_t stream);
int dt_tensor_get(const dt_tensor *t, void *host, size_t offset, size_t n, dt_stream_t stream);

/* Graph op ids for dt_tensor.op (the subset of ggml_op the Flux2 chain
 * emits; numbering is this library's own). */
enum {
    DT_OP_NONE = 0,      /* leaf: data already set */
    DT_OP_ADD, DT_OP_SUB, DT_OP_MUL, DT_OP_DIV,
    DT_OP_SCALE,         /* op_params[0] = float bits */
    DT_OP_SIGMOID, DT_OP_NORM, DT_OP_RMS_NORM, /* norms: op_params[0] = eps bits */
    DT_OP_ROPE,          /* src[1] = pos (I32); op_params: n_dims, mode, base bits, scale bits */
    DT_OP_CONCAT,        /* op_params[0] = dim */
    DT_OP_CPY,           /* cont / cast into dst layout */
    DT_OP_VIEW,          /* data = src[0]->data + byte offset, own ne/nb;
                            offset in op_params[0] (low 32 bits), [1] (high) */
    DT_OP_FILL,          /* op_params[0] = value bits */
    DT_OP_UNARY,         /* op_params[0] = DT_UN_* kind, [1], [2] = p0, p1 bits */
    DT_OP_MUL_MAT,       /* ggml_mul_mat(src0 = weight ne {K, N}, src1 = x ne {K, M1, M2, M3})
                            -> ne {N, M1, M2, M3}; BF16 operands (dt_gemm_bf16),
                            node type BF16 or F32 */
    DT_OP_FLASH_ATTN_EXT,/* ggml_flash_attn_ext(q ne {D, Sq, H, B}, k, v ne {D, Skv, H, B},
                            src[3] = mask, must be NULL) -> ne {D, H, Sq, B};
                            op_params[0] = scale bits; BF16 q/k/v, D = 128 */
    DT_OP_CONV_2D_DIRECT,/* ggml_conv_2d_direct(src0 = weight ne {K, K, Ci, Co} F32/BF16
                            or CONV2D_PACKED,
                            src1 = x ne {W, H, Ci, N} contiguous) -> ne {W', H', Co, N} of
                            x's type; op_params = s0, s1, p0, p1, d0, d1 (stride and
                            dilation 1, K in {1, 3}, padding (K - 1) / 2) */
    DT_OP_UPSCALE,       /* ggml_upscale(x, factor, NEAREST): op_params[0] = factor */
    DT_OP_COUNT
    /* DT_OP_CPY: src[0] is copied (converted) into the node; src[1], when
       set, is the destination tensor the node aliases (ggml_cpy). */
};

/* Execute nodes in order (ggml_backend_graph_compute,
 * src/ggml/ExecutionRuntime.cpp:227, 254).  Before dispatch a fusion pass
 * rewrites the chains listed for the fused entry points above into single
 * kernels when the intermediate nodes are not flagged DT_FLAG_OUTPUT; every
 * other node runs its unfused kernel.  Node data is allocated by the caller
 * (ggml_gallocr's role in the reference, Context.hpp:118-135), except that a
 * VIEW's data is set to its source's data plus its offset when the node is
 * reached, and the nodes the plan absorbs are never read or written.
 *
 * A fused launch reads its inputs and writes the outputs it keeps at its
 * own position, which can differ from node order (a chain reads its first
 * node's inputs at its last node; grouped GEMMs write later nodes' outputs
 * early; see dt_graph_plan_ex).  With flags = 0 (and in dt_graph_compute)
 * the executor therefore replays the plan over the nodes' actual address
 * ranges first, and keeps every launch that would read memory another node
 * has taken over (an allocator that frees after the last reader in node
 * order, like ggml_gallocr, may do that) at its own position, or unfused:
 * any allocation that is valid for the unfused node order is safe.
 * DT_GRAPH_ALLOC_RUNS_AT skips that replay for callers whose allocator
 * already follows dt_graph_plan_ex's runs_at (HipRuntime's arena). */
enum { DT_FLAG_OUTPUT = 1 };
enum { DT_GRAPH_ALLOC_RUNS_AT = 1 };
int dt_graph_compute(dt_backend *be, dt_tensor **nodes, int32_t n_nodes);
int dt_graph_compute_ex(dt_backend *be, dt_tensor **nodes, int32_t n_nodes, uint32_t flags);

/* Run only the fusion pass: fused_into[i] = index of the node whose fused
 * kernel absorbs node i (node i's data is then never read or written, so it
 * needs no allocation, and the fused kernel reads node i's inputs when that
 * root node runs), or -1 when node i runs on its own.  Uses shapes, types,
 * strides, view offsets and flags, never data pointers. */
int dt_graph_plan(dt_tensor **nodes, int32_t n_nodes, int32_t *fused_into);
/* dt_graph_plan plus runs_at[i] = the position in the node list at which node
 * i's kernel runs: i for most nodes, the absorbing node for absorbed ones,
 * and the first member for MUL_MATs grouped into one GEMM launch (those keep
 * their own outputs, which are written at that earlier position).  A caller
 * that allocates node memory places each output at min(i, runs_at[i]) and
 * keeps inputs alive until the runs_at of their last reader. */
int dt_graph_plan_ex(dt_tensor **nodes, int32_t n_nodes, int32_t *fused_into, int32_t *runs_at);
/* The plan dt_graph_compute(_ex with flags = 0) runs for the nodes' current
 * data pointers, without a device: dt_graph_plan_ex after the address-range
 * replay; launches_held = how many launches it held at their position or
 * kept unfused. */
int dt_graph_plan_checked(dt_tensor **nodes, int32_t n_nodes, int32_t *fused_into, int32_t *runs_at,
                          int32_t *launches_held);
/* Statistics of the last dt_graph_compute on this thread: kernels launched
 * and nodes absorbed into fused kernels (_ex: and launches the address-range
 * replay held back). */
int dt_graph_last_stats(int32_t *kernels_launched, int32_t *nodes_fused);
int dt_graph_last_stats_ex(int32_t *kernels_launched, int32_t *nodes_fused, int32_t *launches_held);

/* The launches of one dt_graph_compute recorded as a HIP graph, replayed by
 * dt_graph_exec_launch on the backend's stream: one submission per step
 * instead of the fusion pass plus a launch per kernel (the role of the
 * reference's repeated ggml_backend_graph_compute, ExecutionRuntime.cpp:227,
 * 254).  Call dt_graph_compute on the same nodes once first, so the
 * backend's scratch and RoPE table exist (capture allocates nothing; a
 * capture that would (re)allocate them fails with DT_ERR_INVALID_ARG and
 * keeps nothing).  The
 * replay reads and writes the node data pointers given at capture: inputs
 * are updated in place between replays.  A backend on the NULL stream gets
 * a stream of its own (default priority), used from then on.  The graph
 * records no memset nodes. */
typedef struct dt_graph_exec dt_graph_exec;
int dt_graph_capture(dt_backend *be, dt_tensor **nodes, int32_t n_nodes, dt_graph_exec **out);
/* dt_graph_capture with dt_graph_compute_ex's flags. */
int dt_graph_capture_ex(dt_backend *be, dt_tensor **nodes, int32_t n_nodes, uint32_t flags, dt_graph_exec **out);
/* Refuses (DT_ERR_INVALID_ARG) an exec captured before the backend's scratch
 * or RoPE table was last reallocated: the recorded launches hold their old
 * addresses.  Capture again after such a change. */
int dt_graph_exec_launch(dt_backend *be, dt_graph_exec *exec);
int dt_graph_exec_free(dt_graph_exec *exec);

#ifdef __cplusplus
}
#endif
#endif /* DIT_HIP_H */
