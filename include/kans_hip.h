/*
 * kans_hip.h -- C ABI of the MI355X (gfx950) fused KAN forward library
 * (metal-kans_amd/metal_kans/libkans_hip.so).
 *
 * Plain C: pointers, sizes and ints; no HIP or torch types in any signature
 * (a HIP stream is passed as void*).  Every function returns 0 on success or a
 * negative KANS_ERR_* code (the benchmark helpers return milliseconds, or a
 * negative value on failure); kans_last_error() describes the last failure of
 * the calling thread.  Arguments are validated before any HIP call.
 *
 * The first block mirrors the reference's ctypes surface for the hot path
 * (reference: metal_kans/device.py:64-474, implemented in
 * metal_kans/kernels/metal_kan_bridge.mm); the names, argument order and
 * meaning are kept so the reference's bindings apply unchanged.  The second
 * block is the device-resident layer API that the Python package and the
 * benchmarks use.
 */
#ifndef KANS_HIP_H
#define KANS_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* return codes */
#define KANS_OK 0
#define KANS_ERR_ARG (-1)     /* invalid argument (also the reference quantizers' -1) */
#define KANS_ERR_NODEV (-2)   /* no gfx950 HIP device visible */
#define KANS_ERR_HIP (-3)     /* a HIP runtime call failed */
#define KANS_ERR_STATE (-4)   /* object not ready (e.g. weights not loaded) */
#define KANS_ERR_UNSUPPORTED (-5)

/* basis / dtype codes of the layer API */
#define KANS_BASIS_CHEBY 0
#define KANS_BASIS_RBF 1
#define KANS_BASIS_BSPLINE 2
#define KANS_DT_F32 0
#define KANS_DT_F16 1
#define KANS_DT_BF16 2

const char* kans_last_error(void);

/* ======================================================================= *
 * Reference-named entry points.  Host pointers; blocking unless async mode  *
 * is on (then results land in Y at metal_kan_sync()).  Host weight arrays   *
 * are read on every call, as the reference's zero-copy buffers do.          *
 * ======================================================================= */

/* replaces metal_kan_init (device.py:65-66, metal_kan_bridge.mm:289-404);
 * the shader path is ignored (kernels are compiled ahead of time).
 * Returns -1 when no gfx950 device is visible. */
int metal_kan_init(const char* shader_path);

/* replace metal_kan_set_async / metal_kan_sync (device.py:212-216,
 * metal_kan_bridge.mm:275-287) */
int metal_kan_set_async(int enabled);
int metal_kan_sync(void);

/* replace metal_kan_cheby_forward[_fp16] (device.py:68-72,227-231;
 * metal_kan_bridge.mm:443-530,1890-1971).  K = number of Chebyshev
 * coefficients (the reference's `degree`).  fp16/bf16 arrays are uint16 bit
 * patterns.  The _bf16 variant has no reference counterpart (new dtype). */
int metal_kan_cheby_forward(const float* X, const float* W_cheby, const float* W_base, const float* bias,
                            float* Y, int B, int D_in, int D_out, int K, int has_base, int has_bias);
int metal_kan_cheby_forward_fp16(const uint16_t* X, const uint16_t* W_cheby, const uint16_t* W_base,
                                 const uint16_t* bias, uint16_t* Y, int B, int D_in, int D_out, int K,
                                 int has_base, int has_bias);
int metal_kan_cheby_forward_bf16(const uint16_t* X, const uint16_t* W_cheby, const uint16_t* W_base,
                                 const uint16_t* bias, uint16_t* Y, int B, int D_in, int D_out, int K,
                                 int has_base, int has_bias);

/* replace metal_kan_fastkan_forward[_fp16] (device.py:74-78,233-237;
 * metal_kan_bridge.mm:532-625,1973-2060).  grid = K centres (fp16 bit
 * patterns for _fp16, fp32 for _bf16, as FastKAN keeps its grid fp32 there). */
int metal_kan_fastkan_forward(const float* X, const float* W_rbf, const float* W_base, const float* grid,
                              const float* bias, float* Y, int B, int D_in, int D_out, int K,
                              float inv_denominator, int has_base, int has_bias);
int metal_kan_fastkan_forward_fp16(const uint16_t* X, const uint16_t* W_rbf, const uint16_t* W_base,
                                   const uint16_t* grid, const uint16_t* bias, uint16_t* Y, int B, int D_in,
                                   int D_out, int K, float inv_denominator, int has_base, int has_bias);
int metal_kan_fastkan_forward_bf16(const uint16_t* X, const uint16_t* W_rbf, const uint16_t* W_base,
                                   const float* grid, const uint16_t* bias, uint16_t* Y, int B, int D_in,
                                   int D_out, int K, float inv_denominator, int has_base, int has_bias);

/* replace metal_kan_bspline_forward[_fp16] (device.py:110-114,263-267;
 * metal_kan_bridge.mm:1069-1164,2062-2151).  grid = [grid_min, inv_h] fp32,
 * read on the host; spline_order is ignored (always cubic, G+3 bases). */
int metal_kan_bspline_forward(const float* X, const float* W_spline, const float* W_base, const float* grid,
                              const float* bias, float* Y, int B, int D_in, int D_out, int grid_size,
                              int spline_order, int has_base, int has_bias);
int metal_kan_bspline_forward_fp16(const uint16_t* X, const uint16_t* W_spline, const uint16_t* W_base,
                                   const float* grid, const uint16_t* bias, uint16_t* Y, int B, int D_in,
                                   int D_out, int grid_size, int spline_order, int has_base, int has_bias);
int metal_kan_bspline_forward_bf16(const uint16_t* X, const uint16_t* W_spline, const uint16_t* W_base,
                                   const float* grid, const uint16_t* bias, uint16_t* Y, int B, int D_in,
                                   int D_out, int grid_size, int spline_order, int has_base, int has_bias);

/* replace benchmark_metal_{cheby,fastkan,bspline} (device.py:124-150,
 * metal_kan_bridge.mm:1250-1371): mean wall-clock ms per full host call. */
double benchmark_metal_cheby(const float* X, const float* W_cheby, const float* W_base, const float* bias,
                             float* Y, int B, int D_in, int D_out, int K, int has_base, int has_bias, int warmup,
                             int iters);
double benchmark_metal_fastkan(const float* X, const float* W_rbf, const float* W_base, const float* grid,
                               const float* bias, float* Y, int B, int D_in, int D_out, int K,
                               float inv_denominator, int has_base, int has_bias, int warmup, int iters);
double benchmark_metal_bspline(const float* X, const float* W_spline, const float* W_base, const float* grid,
                               const float* bias, float* Y, int B, int D_in, int D_out, int grid_size,
                               int spline_order, int has_base, int has_bias, int warmup, int iters);

/* replace metal_kan_quantize_int{8,4} (device.py:398-416, metal_kan_bridge.mm:4177-4275).
 * Host (CPU, multi-threaded) quantizers with the rounding of the reference's NumPy fallback
 * (quantization.py:73-99): fp32 division, round half to even.  `weights` is the zero-padded
 * [num_groups * group_size] fp32 matrix; qweight is [num_groups][group_size] (INT8) or
 * [num_groups][group_size/2] (INT4, even index in the low nibble); scales/biases [num_groups]. */
int metal_kan_quantize_int8(const float* weights, uint8_t* qweight, float* scales, float* biases, int num_groups,
                            int group_size);
int metal_kan_quantize_int4(const float* weights, uint8_t* qweight, float* scales, float* biases, int num_groups,
                            int group_size);
/* replace metal_kan_dequantize_int{8,4} (device.py:404-416, metal_kan_bridge.mm:4212-4302):
 * out = fl(fl(q * scale) + bias) on the GPU, bit-identical to quantization.py:136-148. */
int metal_kan_dequantize_int8(const uint8_t* qweight, const float* scales, const float* biases, float* out,
                              int num_groups, int group_size);
int metal_kan_dequantize_int4(const uint8_t* qweight, const float* scales, const float* biases, float* out,
                              int num_groups, int group_size);
/* replace metal_kan_quantize_ternary / metal_kan_dequantize_ternary (device.py:376-379,460-463;
 * metal_kan_bridge.mm:4634-4682,5073-5107).  Quantizer follows quantization.py:231-246
 * (NumPy pairwise fp32 mean of |w| per (row, group)); packed [D_out][ceil(K_dim/16)] uint32,
 * scales [D_out][ceil(K_dim/group_size)]. */
int metal_kan_quantize_ternary(const float* W, uint32_t* packed, float* scales, int D_out, int K_dim,
                               int group_size);
int metal_kan_dequantize_ternary(const uint32_t* packed, const float* scales, float* out, int D_out, int K_dim,
                                 int group_size);
/* replaces metal_kan_swiglu_forward (device.py:431-434, metal_kan_bridge.mm:4846-4875) */
int metal_kan_swiglu_forward(const float* gate, const float* up, float* out, int n);

/* replaces metal_kan_forward_ternary_cheby (device.py:381-385, metal_kan_bridge.mm:4684-4733,
 * fused_kan.metal:2167-2223): fp32 X [B][D_in], ternary W [D_out][D_in*degree] in the packed format
 * above, no base branch, optional fp32 bias; fp32 arithmetic on the exact dequantized weights. */
int metal_kan_forward_ternary_cheby(const float* X, const uint32_t* W_packed, const float* scales,
                                    const float* bias, float* Y, int B, int D_in, int D_out, int degree,
                                    int group_size, int has_bias);

/* replaces metal_kan_chain_pipeline_cheby (device.py:116-122, metal_kan_bridge.mm:1168-1248):
 * fp32 Chebyshev layers dims[0] -> ... -> dims[num_layers], any K per layer (the reference
 * hard-codes K = 4); W_bases[l] / biases[l] may be NULL to disable that branch.  Runs as one
 * replayed HIP graph with device-resident ping-pong activations. */
int metal_kan_chain_pipeline_cheby(const float* X, float* Y, int B, int num_layers, const int* dims,
                                   const int* degrees, const float** W_chebys, const float** W_bases,
                                   const float** biases);

/* Chebyshev layer backward, fp32 host arrays (dY [B][D_out], X [B][D_in], W [D_out][D_in*degree],
 * W_base [D_out][D_in]): dW_cheby, dW_base (has_base), dbias (has_bias) and dX, without a Phi buffer.
 * Replaces metal_kan_cheby_backward_fused (device.py:369-374, metal_kan_bridge.mm:4532-4632) and
 * metal_kan_cheby_backward (device.py:282-287, metal_kan_bridge.mm:2715), which compute the same
 * gradients; T'_k is 0 where |x| > 1 (the clamp), degree <= 32. */
int metal_kan_cheby_backward_fused(const float* dY, const float* X, const float* W_cheby, const float* W_base,
                                   float* dW_cheby, float* dW_base, float* dbias, float* dX, int B, int D_in,
                                   int D_out, int degree, int has_base, int has_bias);
int metal_kan_cheby_backward(const float* dY, const float* X, const float* W_cheby, const float* W_base,
                             float* dW_cheby, float* dW_base, float* dbias, float* dX, int B, int D_in, int D_out,
                             int degree, int has_base, int has_bias);

/* ======================================================================= *
 * Device-resident layer API (no reference counterpart: the reference has   *
 * unified memory and no device-resident objects).                          *
 * ======================================================================= */
typedef struct kans_layer kans_layer;

int kans_init(void);
void* kans_stream(void); /* the library's HIP stream (hipStream_t) */
int kans_synchronize(void);

int kans_layer_create(int basis, int dtype, int D_in, int D_out, int K, int has_base, int has_bias,
                      kans_layer** out);
int kans_layer_destroy(kans_layer* layer);
/* RBF: K centres (fp32) and 1/(2h^2); B-spline: G (K = G + 3), grid_min, inv_h */
int kans_layer_set_rbf(kans_layer* layer, const float* centers, float inv_denominator);
int kans_layer_set_bspline(kans_layer* layer, int grid_size, float grid_min, float inv_h);
/* tiling override for tuning: (wm, nb) in {(64,4),(32,8),(32,4),(32,1)} or (0,0) = automatic; splits >= 0 */
int kans_layer_set_tiling(kans_layer* layer, int wm, int nb, int splits);
/* wave groups per workgroup of the 4-wave fp16/bf16 Chebyshev block kernel, for tuning: 0 = automatic
   (small layers that leave at most one workgroup per CU), 1, 2 or 4 (2 on tiles (32,1) and (32,4), 4 on
   (32,1); elsewhere 1).  The groups split a tile's feature blocks and add their partial sums in a fixed
   order through LDS.  No reference counterpart (the reference has no tiling). */
int kans_layer_set_wave_groups(kans_layer* layer, int groups);
/* 8-wave 16-bit Chebyshev block kernel (one barrier per feature block): 1 (default) holds two feature
   blocks in each LDS stage when both fit (K + has_base <= 5), so one barrier closes two blocks; 0 keeps
   one.  Results are identical.  For tuning and tests; no reference counterpart. */
int kans_layer_set_block_pairs(kans_layer* layer, int on);
int kans_layer_describe(const kans_layer* layer, int B, int* wm, int* nb, int* splits);
/* name of the fused kernel (and its tile) that a forward of batch B runs, NUL-terminated in name[len] */
int kans_layer_kernel(const kans_layer* layer, int B, char* name, int len);
/* as kans_layer_kernel for a forward with X / Y element types x_dtype / y_dtype (each the layer dtype or
 * KANS_DT_F32), naming the template's layer, X and Y types in template order, e.g.
 * "kans::kan_fused_block<_Float16, _Float16, _Float16, BASIS_RBF_REC, 32, 8, 8 waves>" */
int kans_layer_kernel_ex(const kans_layer* layer, int B, int x_dtype, int y_dtype, char* name, int len);
/* weights in the layer dtype: W [D_out][D_in*K] (k fastest), W_base [D_out][D_in], bias [D_out] */
int kans_layer_load_weights(kans_layer* layer, const void* W, const void* W_base, const void* bias);
int kans_layer_load_weights_device(kans_layer* layer, const void* W, const void* W_base, const void* bias);
/* host fp32 weights converted on the device to the layer dtype (round to nearest even) */
int kans_layer_load_weights_f32(kans_layer* layer, const float* W, const float* W_base, const float* bias);
/* device pointers; X [B][ldx] with ldx >= round_up(D_in, 8), ldx % 8 == 0, X 16-byte aligned and
 * columns D_in..ldx-1 finite; Y [B][ldy].  Enqueued on `stream` (NULL = kans_stream()). */
int kans_layer_forward(kans_layer* layer, const void* X, long ldx, void* Y, long ldy, int B, void* stream);
/* as kans_layer_forward with the element types of X and Y chosen separately: each is the layer dtype or
 * KANS_DT_F32 (fp32 activations around a 16-bit layer; fp32 X must be 32-byte aligned) */
int kans_layer_forward_ex(kans_layer* layer, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy,
                          int B, void* stream);
/* host pointers, contiguous [B][D_in] -> [B][D_out] in the layer dtype, pinned staging */
int kans_layer_forward_host(kans_layer* layer, const void* X, void* Y, int B);
/* as kans_layer_forward_host with X in x_dtype: the layer dtype, or KANS_DT_F32 for a 16-bit layer
 * (the input is then used unrounded; weights and MFMA stay 16-bit) */
int kans_layer_forward_host_ex(kans_layer* layer, const void* X, int x_dtype, void* Y, int B);
/* mean ms per device-resident forward, HIP events on the launch stream */
int kans_layer_time_forward(kans_layer* layer, const void* X, long ldx, void* Y, long ldy, int B, int warmup,
                            int iters, float* ms);
/* one timed window after the clock settles: forwards run for at least settle_ms of GPU time, then `iters`
 * forwards are bracketed by stream synchronisation; *wall_ms is the wall-clock mean and *kernel_ms the
 * HIP-event mean over the same launches (so *kernel_ms <= *wall_ms) */
int kans_layer_time_window(kans_layer* layer, const void* X, long ldx, void* Y, long ldy, int B, float settle_ms,
                           int iters, float* kernel_ms, float* wall_ms);

/* multi-layer chain of layers with matching dims and one dtype (no reference counterpart
 * beyond metal_kan_chain_pipeline_cheby): ping-pong device activations kept in fp32 between
 * layers (also for fp16/bf16 layers), host path captured as a HIP graph per batch size.
 * Layers must outlive the chain. */
typedef struct kans_chain kans_chain;
int kans_chain_create(kans_layer** layers, int n, kans_chain** out);
int kans_chain_destroy(kans_chain* chain);
int kans_chain_forward_host(kans_chain* chain, const void* X, void* Y, int B);
/* X in x_dtype: the chain dtype, or KANS_DT_F32 (unrounded input to a 16-bit chain) */
int kans_chain_forward_host_ex(kans_chain* chain, const void* X, int x_dtype, void* Y, int B);
int kans_chain_forward(kans_chain* chain, const void* X, long ldx, void* Y, long ldy, int B, void* stream);
/* mean ms per graph replay (include_copies: also the pinned H2D/D2H copies) */
int kans_chain_time(kans_chain* chain, int B, int warmup, int iters, int include_copies, float* ms);

/* Dense GatedKAN block out = down(SiLU(gate(x)) * up(x)) (gated_kan.py:86-138) on device activations, for
 * layers of one dtype with gate/up d -> h and down h -> d (replaces the reference's four blocking submissions
 * with host round trips between them).  Activations are kept in the block dtype; SwiGLU uses the +-20 clip
 * and the arithmetic of metal_kan_swiglu_forward.  The host path replays one HIP graph per batch size (one
 * H2D and one D2H copy) and honours metal_kan_set_async.  Layers must outlive the block. */
typedef struct kans_gated_dense kans_gated_dense;
int kans_gated_dense_create(kans_layer* gate, kans_layer* up, kans_layer* down, kans_gated_dense** out);
int kans_gated_dense_destroy(kans_gated_dense* block);
/* device X [B][ldx] (x_dtype: block dtype, or fp32 for a 16-bit block), Y [B][ldy] block dtype */
int kans_gated_dense_forward(kans_gated_dense* block, const void* X, int x_dtype, long ldx, void* Y, long ldy, int B,
                             void* stream);
/* host X [B][d] -> Y [B][d] */
int kans_gated_dense_forward_host(kans_gated_dense* block, const void* X, int x_dtype, void* Y, int B);
/* mean ms per graph replay (include_copies: also the pinned H2D / D2H copies) */
int kans_gated_dense_time(kans_gated_dense* block, int B, int warmup, int iters, int include_copies, float* ms);

/* Chebyshev layer backward on device fp32 arrays (no reference counterpart for device pointers; the
 * host form is metal_kan_cheby_backward_fused), enqueued on `stream` (NULL = kans_stream()). */
int kans_cheby_backward(const float* dY, const float* X, const float* W, const float* W_base, float* dW,
                        float* dW_base, float* dbias, float* dX, int B, int D_in, int D_out, int K, int has_base,
                        int has_bias, void* stream);

/* bit-exact dequantizers on device pointers (stream NULL = kans_stream()); bits = 8 or 4 */
int kans_dequantize_affine_device(const void* qweight, const float* scales, const float* biases, float* out,
                                  long num_groups, int group_size, int bits, void* stream);
int kans_dequantize_ternary_device(const uint32_t* packed, const float* scales, float* out, int D_out, int K_dim,
                                   int group_size, void* stream);

/* ----------------------------------------------------------------------- *
 * Quantized KAN layers and the GatedKAN block, fused over the packed        *
 * weights.  Built from the reference's packed formats (quantization.py:13-99 *
 * INT8 / INT4, :191-246 ternary); no reference counterpart for the fused     *
 * forward with the base branch (the reference dequantizes to fp32,           *
 * quantization.py:152-178, gated_kan.py:86-138).  Batches of at most 32 rows *
 * (every format) run the decode GEMVs; larger batches the fused prefill     *
 * kernel, which decodes the packed weights into fp16 MFMA tiles (K and       *
 * basis limits: kans_qlayer_fused; other layers: KANS_ERR_UNSUPPORTED for    *
 * those batches).  Activations are evaluated in fp32 and fed to the MFMAs in *
 * fp16; results are accumulated in fp32.                                     *
 * ----------------------------------------------------------------------- */
typedef struct kans_qlayer kans_qlayer;
/* INT4, group_size 64: qweight [D_out * pad/64][32] uint8, scales / biases [D_out * pad/64] fp32,
 * pad = D_in*K rounded up to 64 (W) or D_in rounded up to 64 (W_base); bias [D_out] of bias_dtype */
int kans_qlayer_create_int4(int D_in, int D_out, int K, int has_base, int has_bias, int group_size,
                            const void* qweight, const float* scales, const float* biases,
                            const void* qweight_base, const float* scales_base, const float* biases_base,
                            const void* bias, int bias_dtype, kans_qlayer** out);
/* INT8, group_size 64: as INT4 with qweight [D_out * pad/64][64] uint8 (quantization.py:88-97) */
int kans_qlayer_create_int8(int D_in, int D_out, int K, int has_base, int has_bias, int group_size,
                            const void* qweight, const float* scales, const float* biases,
                            const void* qweight_base, const float* scales_base, const float* biases_base,
                            const void* bias, int bias_dtype, kans_qlayer** out);
/* ternary, group_size 32: w_packed [D_out][ceil(D_in*K/16)] uint32, scales [D_out][ceil(D_in*K/32)]
 * (base: the same with D_in) */
int kans_qlayer_create_ternary(int D_in, int D_out, int K, int has_base, int has_bias, int group_size,
                               const uint32_t* w_packed, const float* scales, const uint32_t* w_packed_base,
                               const float* scales_base, const void* bias, int bias_dtype, kans_qlayer** out);
int kans_qlayer_destroy(kans_qlayer* layer);
/* The basis expansion of a quantized layer (Chebyshev unless set): the Gaussian RBF with K centres and
 * inv_denominator = 1/(2h^2) (fast_kan.py:40-42; as kans_layer_set_rbf), or the clamped cubic B-spline with
 * G = K - 3 intervals from grid_min, inv_h = G / (max - min) (bspline_kan.py:40-54; as
 * kans_layer_set_bspline).  No reference counterpart: the reference quantizes every layer family's weight
 * matrices (quantization.py:152-178) and runs their fp32 forward on the dequantized weights. */
int kans_qlayer_set_rbf(kans_qlayer* layer, const float* centers, float inv_denominator);
int kans_qlayer_set_bspline(kans_qlayer* layer, int grid_size, float grid_min, float inv_h);
/* 1 when a forward of B rows runs on the fused packed-weight kernels: B <= 32 always (decode GEMVs, every
 * basis and K); larger B when the prefill kernel is built for the layer's K and basis (Chebyshev K <= 9;
 * RBF on uniform centres 2 <= K <= 9 within the recurrence's span guard; B-spline K in {4, 8}; not INT8
 * with the base branch at K = 7, nor INT8 B-spline at K = 8); 0 when such a forward returns
 * KANS_ERR_UNSUPPORTED. */
int kans_qlayer_fused(const kans_qlayer* layer, int B);
/* device pointers; x_dtype / y_dtype any of KANS_DT_* (the prefill path reads fp16 / fp32 X, 16-byte aligned,
 * ldx % 8 == 0 and ldx >= round_up(D_in, 8)) */
int kans_qlayer_forward(kans_qlayer* layer, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy,
                        int B, void* stream);
int kans_qlayer_forward_host(kans_qlayer* layer, const void* X, int x_dtype, void* Y, int y_dtype, int B);

/* GatedKAN block out = down(SiLU(gate(x)) * up(x)) (gated_kan.py:86-138); the layers are borrowed and
 * must outlive the block.  round16: 1 (fp16) / 2 (bf16) rounds the gate, up and hidden activations as a
 * 16-bit model does, 0 keeps them fp32.  Chebyshev layers only (the reference's GatedKAN is built of
 * ChebyKAN layers).  Decode (B <= 32, every format): the gate|up GEMV with SwiGLU into the down layer's
 * basis (computing the basis of x itself at B = 1, after one prep kernel above), the down GEMV and its
 * reduce.  Prefill (larger B, K <= 9; not INT8 at K = 7): one fused launch for gate|up with the SwiGLU epilogue
 * (gate and up columns paired in one tile) writing the hidden activations, one for down. */
typedef struct kans_gated kans_gated;
int kans_gated_create(kans_qlayer* gate, kans_qlayer* up, kans_qlayer* down, kans_gated** out);
int kans_gated_destroy(kans_gated* block);
int kans_gated_forward(kans_gated* block, const void* X, int x_dtype, long ldx, void* Y, int y_dtype, long ldy,
                       int B, int round16, void* stream);
int kans_gated_forward_host(kans_gated* block, const void* X, int x_dtype, void* Y, int y_dtype, int B,
                            int round16);
/* As kans_gated_forward, allocating nothing: every workspace (activation basis, split-K partials, arrival
 * counters, prefill hidden state) is carved from one 64 MiB device array per GPU that the library holds
 * until the process ends.  No counterpart in the reference: for callers that cannot allocate device memory
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  A call whose
 * workspace exceeds 64 MiB returns KANS_ERR_ARG (the config-5 block needs ~49 MB at B = 32).  Calls on one
 * GPU share the array: calls that overlap (other streams or threads) race. */
int kans_gated_forward_noalloc(kans_gated* block, const void* X, int x_dtype, long ldx, void* Y, int y_dtype,
                               long ldy, int B, int round16, void* stream);
/* mean ms per block forward on device X / Y (use_graph: replay one captured HIP graph) */
int kans_gated_time(kans_gated* block, const void* X, int x_dtype, void* Y, int y_dtype, int B, int warmup,
                    int iters, int use_graph, float* ms);
/* mean ms per block forward, replaying one HIP graph per block and cycling through the n blocks (same
 * shapes): with n copies of a block whose weights together exceed the 256 MB MALL, every call streams
 * its weights from HBM (measurement only; no reference counterpart) */
int kans_gated_time_rotate(kans_gated* const* blocks, int n, const void* X, int x_dtype, void* Y, int y_dtype,
                           int B, int warmup, int iters, float* ms);
/* mean ms per block forward of a decode step of the n blocks (d -> d each) captured as one HIP graph, the
 * way a model runs its layers per step: block b reads block b-1's output (X and Y alternate; both device
 * arrays [B][d] of `dtype`), each block streams its own weights (measurement only; no reference
 * counterpart) */
int kans_gated_time_step(kans_gated* const* blocks, int n, void* X, void* Y, int dtype, int B, int warmup, int iters,
                         float* ms);
/* algorithmic bytes of one block forward: packed weights + group parameters + x and y (fp16) */
long long kans_gated_stream_bytes(const kans_gated* block, int B);
/* The GatedKAN block computes SwiGLU(gate, up) and the down layer's basis in one step (on = 1, the
 * default): in the gate|up GEMV's epilogue at B <= 2 (4 launches per block instead of 6), in one
 * kernel after it otherwise (5 instead of 6); on = 0 selects the separate kernels.  Both give
 * identical results.  Returns the previous setting (no reference counterpart: a tuning and test
 * switch). */
int kans_gated_set_fused_swiglu(int on);
/* With the fused SwiGLU epilogue, the gate|up GEMV can compute the basis of x itself, each wave
 * for its own range of the reduction axis in LDS (3 launches per block instead of 4): mode 1 (the
 * default) does so at B = 1, mode 2 at B <= 2, mode 0 never (the separate basis kernel runs
 * first).  All modes give identical results.  Returns the previous mode, or -1 for a mode outside
 * 0..2 (no reference counterpart: a tuning and test switch). */
int kans_decode_set_pre_basis(int mode);
/* Cache policy of the decode path's weight-record loads: 0 automatic (the default), 1 plain, 2
 * non-temporal.  Automatic loads every format's records non-temporally, the faster form when a
 * model's weights stream from HBM on every decode step.
 * Results do not depend on it.  Returns the previous mode, or a negative error code for a mode
 * outside 0..2 (no reference counterpart: a tuning and test switch). */
int kans_decode_set_weight_loads(int mode);
/* Quantized prefill kernel at Chebyshev K = 4 (the GatedKAN shape): 1 (the default) holds two feature
 * blocks in each LDS stage, so one barrier closes two blocks; 0 one block per stage.  Results are
 * identical.  Returns the previous setting, or a negative error code (no reference counterpart: a tuning
 * and test switch). */
int kans_prefill_set_block_pairs(int on);

/* Measured ceilings for the roofline report (no reference counterpart; measurement only).
 * kans_mfma_ceiling: TFLOP/s of back-to-back v_mfma_f32_32x32x16 (dtype DT_F16 / DT_BF16) on 16 A and
 * 16 B operand fragments given as host arrays [16][64 lanes][8 x 16-bit], at the fused block kernel's
 * occupancy; `iters` x 32 MFMAs per wave.  kans_stream_ceiling: GB/s of a read-only streaming kernel
 * over `bytes` of the device buffer `buf` (16-byte aligned), the faster of plain and non-temporal
 * loads. */
int kans_mfma_ceiling(int dtype, const void* a_frags, const void* b_frags, int iters, double* tflops);
int kans_stream_ceiling(const void* buf, size_t bytes, double* gb_per_s);

/* device memory helpers; kans_copy_device is a plain copy kernel (16-byte multiples) used to
 * calibrate hardware byte counters */
int kans_dev_malloc(void** ptr, size_t bytes);
int kans_dev_free(void* ptr);
int kans_memcpy_h2d(void* dst, const void* src, size_t bytes);
int kans_memcpy_d2h(void* dst, const void* src, size_t bytes);
int kans_copy_device(void* dst, const void* src, size_t bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* KANS_HIP_H */
