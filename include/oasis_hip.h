/*
 * oasis_hip.h -- C ABI of liboasis_hip.so, the MI355X (gfx950) implementation of the
 * Oasis-500M DiT denoising step and ViT VAE decoder.
 *
 * Conventions (all entry points):
 *   - Plain device pointers, caller-owned, row-major and contiguous unless a leading
 *     dimension ("ld") is given. Nothing here allocates device memory; everything is
 *     stream-ordered on the given HIP stream (hipStream_t passed as void*, NULL = the
 *     default stream) and may be captured into a hipGraph.
 *   - Return OASIS_OK (0) or a negative OASIS_ERR_* code; oasis_last_error() returns
 *     the message of the last failure on the calling thread.
 *   - dtype codes: OASIS_F32 (fp32) and OASIS_BF16 (bfloat16).
 *
 * Reference citations are paths into zoecarver/open-oasis.
 */
#ifndef OASIS_HIP_H
#define OASIS_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define OASIS_ABI_VERSION 6
#define OASIS_MAX_SUB 64 /* max sub-blocks (2 per DiT block) in one model */

enum {
  OASIS_OK = 0,
  OASIS_ERR_NULL = -1,   /* a required pointer is NULL */
  OASIS_ERR_SHAPE = -2,  /* unsupported or inconsistent shape */
  OASIS_ERR_DTYPE = -3,  /* unsupported dtype code */
  OASIS_ERR_LAUNCH = -4, /* HIP reported an error */
  OASIS_ERR_ARG = -5     /* other invalid argument */
};

enum { OASIS_F32 = 0, OASIS_BF16 = 1 };
enum { OASIS_WEIGHTS_BF16 = 0, OASIS_WEIGHTS_FP8 = 1 };

typedef void* oasis_stream_t;

const char* oasis_last_error(void);
int oasis_abi_version(void);

/* sizeof of the ABI structs, for bindings to check their mirrors: which = 0 epilogue,
 * 1 DiT weights, 2 DiT buffers, 3 VAE weights, 4 VAE buffers; -1 for anything else.
 * No counterpart in the reference (its kernels take ttnn tensors). */
int64_t oasis_abi_struct_size(int which);

/* The fragment-order plan (OASIS_FRAG) for DiT forward passes of `rows` tokens: a mask of 1 QKV,
 * 2 O, 4 FC1, 8 FC2 (whose operand is kept in MFMA fragment order) and 16 (the LayerNorm after O
 * carried into FC1), before a pass narrows it to the weights and buffers it has; 0 above 320 rows.
 * No counterpart in the reference (a tuning query, for benchmarks and tests). */
int oasis_dit_frag_plan(int64_t rows);

/* ======================================================================
 * Reference kernel surface (destination passing: inputs first, outputs last).
 * Elementwise kernels take flat tensors of n elements, all of one dtype.
 * ==================================================================== */

/* out = x * sigmoid(x).  Replaces silu_kernel(x, out)  (src/silu.py:8-9). */
int oasis_silu(const void* x, void* out, int64_t n, int dtype, oasis_stream_t stream);

/* out = x * (scale + 1) + shift.
 * Replaces adaln_modulate_kernel(x, shift, scale, out)  (src/adaln_modulate.py:8-9). */
int oasis_adaln_modulate(const void* x, const void* shift, const void* scale, void* out,
                         int64_t n, int dtype, oasis_stream_t stream);

/* out = residual + x * gate.
 * Replaces gated_residual_kernel(residual, x, gate, out)  (src/gated_residual.py:16-17). */
int oasis_gated_residual(const void* residual, const void* x, const void* gate, void* out,
                         int64_t n, int dtype, oasis_stream_t stream);

/* out = residual + (x + bias) * gate.
 * Replaces bias_gated_residual_kernel(residual, x, bias, gate, out)
 * (src/gated_residual.py:65-66). */
int oasis_bias_gated_residual(const void* residual, const void* x, const void* bias,
                              const void* gate, void* out, int64_t n, int dtype,
                              oasis_stream_t stream);

/* out = (x - mean) / sqrt(var + eps) * weight + bias over the last dim (cols).
 * weight/bias are fp32 whatever dtype is; their rows are read at weight + r*wb_ld (wb_ld = 0 for a [cols] vector,
 * cols for the reference's row-expanded [rows, cols] tensors).
 * Replaces make_layernorm_kernel(dim_tiles)(x, weight, ln_bias, scaler, mean_scale, out)
 * (src/layernorm.py:15-17; instance layernorm_d1024, oasis_inference.py:172).
 * scaler/mean_scale are Tensix reduction constants and have no counterpart here. */
int oasis_layernorm(const void* x, const void* weight, const void* bias, int64_t wb_ld,
                    void* out, int64_t rows, int64_t cols, float eps, int dtype,
                    oasis_stream_t stream);

/* out[M,N] = x[M,K] @ w.  w_layout 0: w is [K,N] (the reference layout), 1: w is [N,K].
 * x and w are bf16; out is fp32 or bf16 (out_dtype).
 * Replaces make_linear_kernel(k_chunk)(x, w, out)  (src/linear.py:10-12; instance
 * linear_k32, oasis_inference.py:171). */
int oasis_linear(const void* x, const void* w, void* out, int64_t M, int64_t K, int64_t N,
                 int w_layout, int out_dtype, oasis_stream_t stream);

/* out[r, :] = silu_cond[0, :] @ w[K,N] + b[N] for r in [0, out_rows) (row expansion).
 * All fp32 except w (bf16).
 * Replaces make_adaln_matmul_expand_kernel(k_tiles, n_repeat)(silu_cond, adaln_w,
 * adaln_b, out)  (src/adaln_matmul_expand.py:13-15). */
int oasis_adaln_matmul_expand(const float* silu_cond, const void* w, const float* b,
                              float* out, int64_t K, int64_t N, int64_t out_rows,
                              oasis_stream_t stream);

/* RoPE on the Q and K columns of qkv plus head split.
 *   qkv:  [rows, ld_qkv], Q at cols [0,D), K at [D,2D), V at [2D,3D), D = n_heads*64.
 *         Extra columns (the reference's Q_swap/K_swap) are ignored: the pair swap of
 *         rotate_half is done in registers.
 *   cos/sinp: fp32 tables; the value for row r, head h, dim d is at
 *         tab[pos*tab_ld + h*tab_head_stride + d] with pos = (r / pos_div) % pos_mod.
 *         sinp carries the rotate_half sign (-sin at even d, +sin at odd d).
 *   mode 0 (heads-first): out row (f*n_heads + h)*seq + p for r = f*seq + p
 *         (spatial / VAE layout, make_rope_layout_kernel and make_vae_rope_kernel);
 *   mode 1 (token-major): out row r, cols h*64..h*64+63 (make_rope_temporal_kernel).
 *   dtype applies to qkv and the three outputs; head_dim must be 64.
 * Replaces make_rope_layout_kernel(...)(qkv_full, cos_tab, sin_tab, q_out, k_out, v_out)
 * (src/rope_layout_kernel.py:16-22), make_rope_temporal_kernel(...)(same)
 * (src/rope_layout_kernel.py:89-97) and make_vae_rope_kernel(...)(same)
 * (src/vae_rope.py:8-10). */
int oasis_rope_layout(const void* qkv, int64_t ld_qkv, const float* cos, const float* sinp,
                      int64_t tab_ld, int64_t tab_head_stride, int64_t pos_div,
                      int64_t pos_mod, void* q_out, void* k_out, void* v_out, int64_t rows,
                      int64_t seq, int64_t n_heads, int64_t head_dim, int mode, int dtype,
                      oasis_stream_t stream);

/* Multi-head attention with heads stacked along rows:
 *   Q,out: [n_heads_total*sq, head_dim]; K,V: [n_heads_total*skv, head_dim].
 *   out = softmax(Q K^T * scale + bias) V per head; bias is an optional fp32
 *   [sq, skv] additive mask shared by all heads (NULL for none); causal != 0 masks
 *   keys j > i. dtype applies to Q, K, V and out; head_dim must be 64.
 * Replaces make_sdpa_kernel(...)(Q_all, K_all, V_all, scaler, attn_scratch, out)
 * (src/sdpa.py:27-41) and make_sdpa_causal_kernel(...)(Q_all, K_all, V_all, scaler,
 * bias, attn_scratch, out) (src/sdpa_causal.py:17-23). */
int oasis_sdpa(const void* Q, const void* K, const void* V, void* out, int64_t n_heads_total,
               int64_t sq, int64_t skv, int64_t head_dim, float scale, const float* bias,
               int causal, int dtype, oasis_stream_t stream);

/* ======================================================================
 * Hot-path building blocks (used by the composite entry points below).
 * ==================================================================== */

enum {
  OASIS_EPI_STORE_F32 = 0,    /* out_f32[m, n] = acc + bias                        */
  OASIS_EPI_STORE_BF16 = 1,   /* out_bf16[m, n] = acc + bias                       */
  OASIS_EPI_GELU_TANH = 2,    /* out_bf16[m, n] = gelu_tanh(acc + bias)            */
  OASIS_EPI_GELU_ERF = 3,     /* out_bf16[m, n] = gelu_erf(acc + bias)             */
  OASIS_EPI_GATED_RES = 4,    /* out_f32[m, n] += gate[f(m), n] * (acc + bias)     */
  OASIS_EPI_RESIDUAL = 5,     /* out_f32[m, n] += acc + bias                       */
  OASIS_EPI_QKV_ROPE = 6,     /* RoPE on Q,K + head split into q/k/v (bf16)         */
  OASIS_EPI_UNPATCHIFY = 7,   /* VAE predictor -> clamp(-1,1) CHW frames (fp32): rows of
                                 frame f (rows_per_frame each) to out_f32 + f*3*H*W     */
  OASIS_EPI_PARTIAL_F32 = 8,  /* split-K slice s: out_f32[s*split_stride + m*ld_out + n] = acc
                                 (no bias; summed by oasis_residual_ln)                */
  OASIS_EPI_GELU_TANH_FP8 = 9,/* g = gelu_tanh(acc + bias) as fp8 activation blocks:
                                 out_fp8[m*ld_out + n] = e4m3(g / 2^e) and
                                 out_scale[m*ld_scale + n/32] = e + 127 per 32 columns
                                 (N % 32 == 0); the A operand of oasis_gemm_fp8_a8     */
  OASIS_EPI_GELU_TANH_FRAG = 10,/* gelu_tanh(acc + bias) into out_bf16 in MFMA fragment order
                                 (below) as a matrix of ld_out columns (ld_out % 32 == 0):
                                 the A operand of oasis_gemm_bf16_frag                  */
  /* The pair below carries a LayerNorm + modulate from one product into the next, so that
   * (with f = f(m), s = mod_scale[f], t = mod_shift[f])
   *   GELU_TANH_LN(GATED_RES_LN(...)) = gelu_tanh((LN(x_new) * s + t) @ B^T + bias)
   * without the normalised rows ever being formed. oasis_gemm_bf16_frag only.            */
  OASIS_EPI_GATED_RES_LN = 11,/* x = out_f32[m, n] += gate[f, n] * (acc + bias[n]) (N % 32 == 0);
                                 y = x - ln_center[m]; out_bf16 (fragment order, ld_out
                                 columns) = y * mod_scale[f, n]; ln_stats[m][n/G] = (sum of
                                 y, sum of y^2) over groups of G columns (G = 32 when its
                                 tiles are 32 columns wide or more, else 16); ln_mod rows
                                 2f, 2f + 1 = bf16(mod_scale[f]), bf16(mod_shift[f]) for the
                                 frames f < ceil(M / rows_per_frame) <= 8                  */
  OASIS_EPI_GELU_TANH_LN = 12 /* A = a GATED_RES_LN output over K = its N (K <= 1024, one
                                 split): gelu_tanh(r (acc - mu c1[f, n]) + c2[f, n] + bias[n])
                                 with mu, r = 1/sqrt(var + ln_eps) from ln_stats[m][0..K/G),
                                 c1 and c2 = ln_mod rows 2f and 2f + 1 @ B^T; into out_bf16,
                                 in fragment order when out_frag                          */
};

/* MFMA fragment order of a bf16 matrix X [R, C] (R % 16 == 0, C % 32 == 0): R/16 x C/32
 * blocks of 512 elements, block (rb, s) at element (rb*C/32 + s)*512; within a block 64
 * pieces of 8 elements, piece l = X[16*rb + l%16][32*s + 8*(l/16) .. +7]: the operand lane l
 * of v_mfma_f32_16x16x32_bf16 takes, so a wave reads a block as one contiguous 1 KB load.
 * (The 16-row tile order of oasis_gemv_bf16_tiled is the same layout.) */

/* Row m is token p of frame f = m / rows_per_frame (p = m % rows_per_frame);
 * frame f is frame t = f % frames_per_stream of stream b = f / frames_per_stream. */
typedef struct {
  int kind;
  int n_heads;              /* QKV_ROPE: heads (head_dim is 64)                   */
  const float* bias;        /* [N] fp32 or NULL                                   */
  float* out_f32;           /* STORE_F32 / GATED_RES / RESIDUAL / UNPATCHIFY      */
  void* out_bf16;           /* STORE_BF16 / GELU_*                                */
  int64_t ld_out;           /* leading dimension of out_* (elements)              */
  const float* gate;        /* GATED_RES: gate row of frame f at gate + f*gate_fstride */
  int64_t gate_fstride;
  int64_t rows_per_frame;
  int64_t frames_per_stream;
  /* QKV_ROPE: element offset of (b, t, p, h, d) = b*s_b + t*s_t + p*s_p + h*s_h + d
   * in each of q/k/v; RoPE position = t if rope_by_frame else p; tables [pos][64]. */
  void* q;
  void* k;
  void* v;
  const float* rope_cos;
  const float* rope_sinp;
  int rope_by_frame;
  int unpatch_grid_w;       /* UNPATCHIFY: patches per row of the latent grid      */
  int64_t s_b, s_t, s_p, s_h;
  int unpatch_patch;        /* UNPATCHIFY: patch edge (20)                         */
  int unpatch_channels;     /* UNPATCHIFY: channels (3)                            */
  int64_t split_stride;     /* PARTIAL_F32: elements between split-K slices         */
  void* out_fp8;            /* GELU_TANH_FP8: e4m3 bytes, row stride ld_out         */
  void* out_scale;          /* GELU_TANH_FP8: e8m0 block scales, row stride ld_scale */
  int64_t ld_scale;
  const float* mod_scale;   /* GATED_RES_LN: modulate scale (+1) row of frame f at mod_scale + f*gate_fstride */
  const float* mod_shift;   /* GATED_RES_LN: modulate shift rows, the same stride     */
  const float* ln_center;   /* GATED_RES_LN: [M], subtracted before the statistics    */
  float* ln_stats;          /* *_LN: [M][N/G][2], G 16 or 32 (GATED_RES_LN's N = GELU_TANH_LN's K;
                               [M][N/16][2] always holds them) */
  void* ln_mod;             /* *_LN: bf16 [16, N] in fragment order (rows 2f, 2f + 1)  */
  float ln_eps;             /* GELU_TANH_LN                                           */
  int out_frag;             /* GELU_TANH_LN: out_bf16 in fragment order              */
} oasis_epilogue_t;

/* acc[M,N] = A[M,K] @ B[N,K]^T (bf16 in, fp32 accumulate) followed by the epilogue.
 * K % 64 == 0, N % 8 == 0, lda and ldb below 2^22 elements. */
int oasis_gemm_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M,
                    int64_t N, int64_t K, const oasis_epilogue_t* epi, oasis_stream_t stream);

/* Same with an explicit tile configuration (0..12, the kTiles table of gemm.hip; -1 = default) and
 * split-K count (splits divides K/64; splits > 1 requires OASIS_EPI_PARTIAL_F32). The wave-split
 * tiles 8..12 need K/splits = 256, 512, 1024 or 2048 and refuse OASIS_EPI_GELU_TANH_FP8.
 * No counterpart in the reference: it exposes the tiling for tuning and benchmarks. */
int oasis_gemm_bf16_config(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M,
                           int64_t N, int64_t K, const oasis_epilogue_t* epi, int tile, int splits,
                           oasis_stream_t stream);

/* acc[M,N] = A[M,K] @ B[N,K]^T with both operands in MFMA fragment order: A [a_rows, K] (a_rows
 * >= M rounded up to the tile: 48 rows for M <= 160, else 80; rows past M are read and their
 * results dropped), B [N, K]. Each workgroup's 8 waves split its K slice, every load issued
 * before the first MFMA, the partial tiles summed through LDS. M % 16 == 0, M <= 320,
 * N % 16 == 0, K % 256 == 0 and K/splits one of 256, 512, 1024 (splits > 1 requires
 * OASIS_EPI_PARTIAL_F32). Any epilogue but UNPATCHIFY and GELU_TANH_FP8.
 * No counterpart in the reference: it is the DiT projections' kernel at one or two frames. */
int oasis_gemm_bf16_frag(const void* A, int64_t a_rows, const void* B, int64_t M, int64_t N, int64_t K,
                         const oasis_epilogue_t* epi, int splits, oasis_stream_t stream);

/* fp8 weight GEMM: acc[M,N] = A[M,K] @ (Bq[N,K] * w_scale[N])^T, then the epilogue.
 * A bf16 (quantized per 32-wide K block to e4m3 with a power-of-two scale inside the kernel),
 * Bq OCP fp8 e4m3 bytes, w_scale fp32 per output channel. K % 128 == 0, N % 8 == 0,
 * lda % 8 == 0, ldb % 16 == 0, both below 2^22. tile: 0..4 (gemm_fp8.hip's kTiles8), -1 = default;
 * splits divides K/128 (> 1 requires OASIS_EPI_PARTIAL_F32).
 * No counterpart in the reference: it has no sub-fp32 weight path (the config-4 serving
 * case of the build's benchmark plan). */
int oasis_gemm_fp8(const void* A, int64_t lda, const void* Bq, int64_t ldb, const float* w_scale, int64_t M,
                   int64_t N, int64_t K, const oasis_epilogue_t* epi, int tile, int splits,
                   oasis_stream_t stream);

/* Same product with the A operand already in fp8 activation blocks: A8 e4m3 bytes [M, lda]
 * (lda % 16 == 0) and A_scale e8m0 bytes [M, lds] (lds >= K/32, lds % 4 == 0), one scale per
 * 32-wide K block (as oasis_quantize_act_fp8 and OASIS_EPI_GELU_TANH_FP8 write them).
 * No counterpart in the reference (see oasis_gemm_fp8). */
int oasis_gemm_fp8_a8(const void* A8, int64_t lda, const void* A_scale, int64_t lds, const void* Bq,
                      int64_t ldb, const float* w_scale, int64_t M, int64_t N, int64_t K,
                      const oasis_epilogue_t* epi, int tile, int splits, oasis_stream_t stream);

/* bf16 activations x[M, K] (K % 32 == 0) -> fp8 blocks: for each 32-wide block of a row,
 * e = floor(log2(max |x|)) - 7 (clamped at -127), q = e4m3(x / 2^e) (nearest even) and
 * scale byte e + 127. No counterpart in the reference (see oasis_gemm_fp8). */
int oasis_quantize_act_fp8(const void* x, int64_t ldx, int64_t M, int64_t K, void* q, int64_t ldq,
                           void* scale, int64_t lds, oasis_stream_t stream);

/* Per-output-channel e4m3 quantization of a bf16 weight W[N,K] (K % 8 == 0):
 * scale[n] = max_k |W[n,k]| / 448 (1 for an all-zero row), q[n,k] = round_e4m3(W[n,k] / scale[n]),
 * round to nearest even. No counterpart in the reference (see oasis_gemm_fp8). */
int oasis_quantize_fp8_rows(const void* W, int64_t N, int64_t K, void* q, float* scale,
                            oasis_stream_t stream);

/* y_bf16[m, :] = LN(x[m, :]) * scale_p1[f(m), :] + shift[f(m), :], f(m) = m / rows_per_frame,
 * frame rows of shift/scale_p1 at + f*ada_fstride.  scale_p1 already holds (1 + scale).
 * LN has no affine, eps as given.  (ttnn.layer_norm + addcmul,
 * oasis_inference.py:1053-1056,1168-1171.) */
int oasis_ln_modulate(const float* x, int64_t M, int64_t D, const float* shift,
                      const float* scale_p1, int64_t ada_fstride, int64_t rows_per_frame,
                      void* y_bf16, float eps, oasis_stream_t stream);

/* Residual update fused with the next LayerNorm, one pass over each row:
 *   if n_partials > 0: x[m, :] += g(m) * (sum_s partial[s*partial_stride + m*D + :] + bias)
 *       g(m) = gate[f(m)*gate_fstride + :] (gate != NULL) or 1; f(m) = m / rows_per_frame;
 *   if y_bf16 != NULL: y_bf16[m, :] = LN(x[m, :]) * ln_a[f(m)*ln_fstride + :] + ln_b[...]
 *       (modulation: ln_a = scale_p1 and ln_b = shift rows; affine: ln_fstride = 0).
 * n_partials in {0..4, 8}; D in {256, 512, 1024, 2048}. The partials are the split-K
 * slices of an OASIS_EPI_PARTIAL_F32 GEMM. (O / FC2 bias + gated residual + the next
 * LN + modulate, oasis_inference.py:1153-1171,1191-1201,1053-1056; VAE residual + LN,
 * oasis_inference.py:1584-1611.) */
int oasis_residual_ln(float* x, int64_t M, int64_t D, const float* partial, int n_partials,
                      int64_t partial_stride, const float* bias, const float* gate,
                      int64_t gate_fstride, int64_t rows_per_frame, const float* ln_a,
                      const float* ln_b, int64_t ln_fstride, void* y_bf16, float eps,
                      oasis_stream_t stream);

/* y_bf16 = LN(x) * w + b (affine LayerNorm of the VAE, oasis_inference.py:1559,1592,1611). */
int oasis_ln_affine(const float* x, int64_t M, int64_t D, const float* w, const float* b,
                    void* y_bf16, float eps, oasis_stream_t stream);

/* Non-causal multi-head attention, heads-first inputs, token-major output:
 *   q,k,v: bf16 [n_frames*n_heads, L, 64]; out: bf16 [n_frames*L, n_heads*64].
 * (spatial SDPA, src/sdpa.py; VAE SDPA, oasis_inference.py:1575-1577.) */
int oasis_attention(const void* q, const void* k, const void* v, void* out, int64_t n_frames,
                    int64_t L, int64_t n_heads, float scale, oasis_stream_t stream);

/* Causal attention over the T frames of each (stream, position, head) group:
 *   q,k,v: bf16 [B, P, n_heads, T, 64]; out: bf16 [B*T*P, n_heads*64] token-major.
 * (temporal SDPA, src/sdpa_causal.py with the bias of oasis_inference.py:843-857.) */
int oasis_temporal_attention(const void* q, const void* k, const void* v, void* out,
                             int64_t B, int64_t T, int64_t P, int64_t n_heads, float scale,
                             oasis_stream_t stream);

/* oasis_attention and oasis_temporal_attention writing their output as fp8 activation blocks
 * (e4m3 bytes out8 [rows, n_heads*64], e8m0 scales out8_scale [rows, n_heads*2]): the bytes
 * oasis_quantize_act_fp8 would make of the bf16 output, in the same launch. The fp8-weight
 * step's O projection reads them. (No counterpart in the reference, whose attention output is
 * bf16; it fuses the fp8 path's activation quantization, config 4.) */
int oasis_attention_fp8(const void* q, const void* k, const void* v, void* out8, void* out8_scale,
                        int64_t n_frames, int64_t L, int64_t n_heads, float scale, oasis_stream_t stream);
int oasis_temporal_attention_fp8(const void* q, const void* k, const void* v, void* out8, void* out8_scale,
                                 int64_t B, int64_t T, int64_t P, int64_t n_heads, float scale,
                                 oasis_stream_t stream);

/* Temporal sub-block front half for a two-frame window in one launch: QKV projection,
 * temporal RoPE and causal attention over the frames of each (stream, position, head).
 *   h: bf16 LN output [B*T*P, ldh] (row (b*T + t)*P + p); w_qkv: bf16 [3D, D], D = 64 n_heads;
 *   out: bf16 [B*T*P, D] token-major attention output; t_cos / t_sinp: fp32 temporal RoPE
 *   tables [>= 2][64] (row = RoPE position, sinp with the rotate_half sign);
 *   k_cache / v_cache: bf16 [B][P][n_heads][2][64] or both NULL.
 * T = 2: both frames (positions 0, 1); query frame 0 attends to its own key, query frame 1 to
 *   both. With a cache, slot t receives frame t's rotated K and its V.
 * T = 1: the current frame at RoPE position 1 attends to cache slot 0 (the context frame's
 *   rotated K and V) and to itself; the cache is read only.
 * q, k and v are rounded to bf16 before the attention, as oasis_temporal_attention sees them.
 * P must be a multiple of 16. (run_sub_block's temporal qkv linear + rope_temporal +
 * sdpa_causal, oasis_inference.py:1060-1151, and run_sub_block_t1's, oasis_inference.py:
 * 1218-1352.) */
int oasis_temporal_qkv_attention(const void* h, int64_t ldh, const void* w_qkv, void* out, int64_t B,
                                 int64_t T, int64_t P, int64_t n_heads, const float* t_cos,
                                 const float* t_sinp, void* k_cache, void* v_cache, float scale,
                                 oasis_stream_t stream);

enum { OASIS_ACT_NONE = 0, OASIS_ACT_SILU = 1, OASIS_ACT_TEMB = 2 };

/* Skinny GEMM for R <= 1024 rows (one pass over W per 16 rows):
 * out[r, n] (+)= act_out(sum_k act_in(x[r, k]) W[n, k] + b[n]).
 * x fp32 [R, ldx], W bf16 [N, K] (K % 64 == 0), b fp32 [N] or NULL, out fp32 [R, ld_out].
 * x is split into bf16 hi + lo parts, so the product keeps ~16 mantissa bits of x.
 * accumulate != 0 adds into out. (adaLN GEMMs, oasis_inference.py:983-993, and the
 * conditioning MLP, oasis_inference.py:1406-1427.) */
int oasis_gemv_bf16(const float* x, int64_t ldx, int64_t R, const void* W, int64_t N,
                    int64_t K, const float* b, float* out, int64_t ld_out, int act_in,
                    int act_out, int accumulate, oasis_stream_t stream);

/* Same product with W in 16-row MFMA tile order: for tile t (rows 16t..16t+15) and each
 * 32-wide K step s, 64 pieces of 8 bf16 back to back, piece l holding row 16t + (l & 15),
 * columns 32s + 8(l >> 4) .. +7 (tile t, step s at element offset (t*K/32 + s)*512). Each
 * wave's weight loads are then 1 KB contiguous. The DiT's stacked adaLN weights (ada_w of
 * oasis_dit_weights_t) are kept in this order. No counterpart in the reference: a storage
 * order of the adaLN projections' weights (oasis_inference.py:983-993). */
int oasis_gemv_bf16_tiled(const float* x, int64_t ldx, int64_t R, const void* W, int64_t N,
                          int64_t K, const float* b, float* out, int64_t ld_out, int act_in,
                          int act_out, int accumulate, oasis_stream_t stream);

/* The same product with fp32 weights and fp32 arithmetic throughout:
 * out[r, n] (+)= act_out(sum_k act_in(x[r, k]) W[n, k] + b[n]), W fp32 [N, K] (K % 4 == 0,
 * K <= 4096), R <= 1024. act_in = OASIS_ACT_TEMB: x is fp32 [R, ldx] with one timestep per
 * row (x[r*ldx]) and the row multiplied is its embedding [cos(t f_i), sin(t f_i)],
 * f_i = exp(-ln(10000) i / (K/2)) (timestep_embedding, oasis_inference.py:307-311).
 * (The projections the reference keeps in fp32: the conditioning MLP and action projection,
 * oasis_inference.py:512-520,1406-1427, and the final layer's adaLN,
 * oasis_inference.py:527-532,1499-1511.) */
int oasis_gemv_f32(const float* x, int64_t ldx, int64_t R, const float* W, int64_t N,
                   int64_t K, const float* b, float* out, int64_t ld_out, int act_in,
                   int act_out, int accumulate, oasis_stream_t stream);

/* out[r, :] = [cos(t_r f), sin(t_r f)], f_i = exp(-ln(10000) i / (dim/2)), dim even.
 * (timestep_embedding, oasis_inference.py:307-311.) */
int oasis_timestep_embedding(const float* t, int64_t R, int64_t dim, float* out,
                             oasis_stream_t stream);

/* out[m, n] = b[n] + sum_k x[m, k] W(n, k) in fp32 (K <= 256; w_dtype OASIS_F32 or OASIS_BF16;
 * w_layout 0: W is [N, K], 1: W is [K, N]), for the small-K projections: patch embed (K=64, the
 * reference's fp32 W_rt [64, D], oasis_inference.py:1821-1826,1911) and the VAE post_quant
 * linear (K=32, bf16, oasis_inference.py:686-690,1551). */
int oasis_small_linear(const float* x, int64_t ldx, int64_t M, int64_t K, const void* W,
                       int w_dtype, int w_layout, int64_t N, const float* b, float* out,
                       int64_t ld_out, oasis_stream_t stream);

/* chunk <- c4*x0 + c5*eps with x0 = c0*chunk - c1*v, eps = (c2*chunk - x0)*c3, n elements.
 * (DDIM update, oasis_inference.py:1919-1931.) */
int oasis_ddim_update(float* chunk, const float* v, int64_t n, float c0, float c1, float c2,
                      float c3, float c4, float c5, oasis_stream_t stream);

/* DiT patch rows [gh*gw, 4*C] (cols (p,q,c)) -> VAE latent [(2gh)*(2gw), out_cols] scaled by
 * inv_scale, channels in cols [0, C), zeros after.
 * (bridge_unpatchify, oasis_inference.py:1651-1709.) */
int oasis_bridge(const float* chunk, float* latent, int64_t gh, int64_t gw, int64_t C,
                 int64_t out_cols, float inv_scale, oasis_stream_t stream);

/* [gh*gw, 3*ps*ps] patches (cols (c,p,q)) -> clamp([3, gh*ps, gw*ps], -1, 1).
 * (vae_unpatchify + clamp, oasis_inference.py:1636-1645,2292.) */
int oasis_vae_unpatchify(const float* patches, float* frame, int64_t gh, int64_t gw,
                         int64_t ps, oasis_stream_t stream);

/* out[i] = clamp(z_i, -clamp_abs, clamp_abs), i < n, z_i N(0, 1) draws (Philox4x32-10 under key
 * seed, counter block (i / 4, *counter), Box-Muller); copy, if not NULL, gets the same values.
 * *counter (device memory) is then incremented, so a captured graph draws new noise on every
 * replay. The interactive loop's per-frame noise (play.py:466-472, torch.randn clamped to +-20),
 * drawn inside the frame graph. */
int oasis_noise_normal(float* out, float* copy, int64_t n, uint64_t seed, uint32_t* counter,
                       float clamp_abs, oasis_stream_t stream);

/* [C, H, W] frame in [-1, 1] -> [H, W, C] in [0, 1]: (x + 1) / 2, clamped. The interactive loop's
 * frame for display (play.py:476-480). */
int oasis_frame_hwc(const float* frame, float* out, int64_t C, int64_t H, int64_t W,
                    oasis_stream_t stream);

/* ======================================================================
 * Composite entry points: the DiT step, the VAE decoder and the DDIM frame.
 * ==================================================================== */

/* Device pointers of one DiT ([out, in] weights; biases and tables fp32).
 * Sub-block j = 2*i + (0 spatial | 1 temporal) of block i.
 * ada_w/ada_b (bf16 / fp32) hold every sub-block's adaLN projection back to back: rows
 * [j*6D, (j+1)*6D) for sub-block j, with +1 folded into the bias of each scale chunk; ada_w is
 * stored in the 16-row tile order of oasis_gemv_bf16_tiled.
 * The pieces the reference keeps in fp32 are fp32 here too: the conditioning MLP and action
 * projection (oasis_inference.py:512-520), the patch embed W_rt (1821-1826), and the final
 * layer's adaLN and linear (527-532). The adaLN rows of all consumers go to one buffer of
 * width n_sub*6D + 2D: sub-block j at column j*6D, the final layer at n_sub*6D. */
typedef struct {
  int n_sub;                 /* 2 * blocks                                         */
  int d_model;               /* 1024                                               */
  int n_heads;               /* 16 (head_dim 64)                                   */
  int d_mlp;                 /* 4096                                               */
  int grid_h, grid_w;        /* 9 x 16 patches                                     */
  int patch_dim;             /* 64 = 2*2*16                                        */
  int freq_dim;              /* 256                                                */
  int ext_dim_pad;           /* 64 (25 action dims zero-padded)                    */
  const void* ada_w;         /* [n_sub*6D, D] bf16, 16-row tile order              */
  const float* ada_b;        /* [n_sub*6D]                                         */
  const float* final_ada_w;  /* [2D, D] fp32: shift, scale                         */
  const float* final_ada_b;  /* [2D], +1 folded into the scale half                */
  const void* qkv_w[OASIS_MAX_SUB];   /* [3D, D], no bias                          */
  const void* out_w[OASIS_MAX_SUB];   /* [D, D]                                    */
  const float* out_b[OASIS_MAX_SUB];
  const void* fc1_w[OASIS_MAX_SUB];   /* [Dm, D]                                   */
  const float* fc1_b[OASIS_MAX_SUB];
  const void* fc2_w[OASIS_MAX_SUB];   /* [D, Dm]                                   */
  const float* fc2_b[OASIS_MAX_SUB];
  const float* final_w;      /* [64, D] fp32                                       */
  const float* final_b;
  const float* xemb_w;       /* [64, D] fp32 patch embed (K-major), rows in (p, q, c) order */
  const float* xemb_b;
  const float* temb_w0;      /* [D, 256] fp32                                      */
  const float* temb_b0;
  const float* cond_w;       /* [D, D + ext_dim_pad] fp32: the MLP's second linear in
                                cols [0, D), the action projection in [D, D + ext_dim_pad) */
  const float* cond_b;       /* [D]: the sum of their two biases                   */
  const float* s_cos;        /* [grid_h*grid_w, 64] spatial RoPE (sin with sign)  */
  const float* s_sinp;
  const float* t_cos;        /* [t_max, 64] temporal RoPE                          */
  const float* t_sinp;
  int t_max;
  /* OASIS_WEIGHTS_BF16: qkv_w/out_w/fc1_w/fc2_w are bf16. OASIS_WEIGHTS_FP8: they are e4m3
   * bytes ([out, in], from oasis_quantize_fp8_rows) with fp32 per-output-channel scales in
   * qkv_s/out_s/fc1_s/fc2_s, and the four projections run on oasis_gemm_fp8. */
  int weight_format;
  const float* qkv_s[OASIS_MAX_SUB];
  const float* out_s[OASIS_MAX_SUB];
  const float* fc1_s[OASIS_MAX_SUB];
  const float* fc2_s[OASIS_MAX_SUB];
  /* OASIS_WEIGHTS_BF16 only, optional, per role: the projection weights once more in MFMA
   * fragment order (see above). A forward pass of at most 320 tokens (a multiple of 48), with
   * frag_rows in the buffers, keeps the operand of each role the library's plan picks for its
   * size (by default O's and FC2's up to 160 tokens, O's above; OASIS_FRAG="m1[,m2]" sets the
   * masks, bits 1 QKV, 2 O, 4 FC1, 8 FC2) in fragment order and runs that projection on
   * oasis_gemm_bf16_frag, when every sub-block of the pass has that role's weights here. NULL
   * keeps the role on the row-major weights. */
  const void* qkv_wf[OASIS_MAX_SUB];
  const void* out_wf[OASIS_MAX_SUB];
  const void* fc1_wf[OASIS_MAX_SUB];
  const void* fc2_wf[OASIS_MAX_SUB];
} oasis_dit_weights_t;

/* Activation workspace for up to max_rows = B*T*P tokens (caller-allocated). */
typedef struct {
  int64_t max_rows;
  float* x;        /* [max_rows, D] fp32 residual stream                          */
  void* h;         /* [max_rows, D] bf16 normalised + modulated                   */
  void* q;         /* [max_rows, D] bf16 each                                     */
  void* k;
  void* v;
  void* attn;      /* [max_rows, D] bf16                                          */
  void* mlp;       /* [max_rows, Dm] bf16                                         */
  float* partial;  /* [max_splits, max_rows, D] fp32 split-K slices               */
  int64_t max_splits;
  /* fp8 weights only (NULL otherwise): the projections' A operands as fp8 activation
   * blocks (e4m3 bytes + one e8m0 scale per 32 columns) */
  void* act8;        /* [max_rows, D] e4m3: LN outputs and the attention output     */
  void* act8_scale;  /* [max_rows, D/32] e8m0                                       */
  void* mlp8;        /* [max_rows, Dm] e4m3: GELU(FC1) output                       */
  void* mlp8_scale;  /* [max_rows, Dm/32] e8m0                                      */
  /* rows h, attn and mlp hold (>= max_rows), for the fragment-order passes (0: none). A pass of
   * M <= 320 tokens needs M rounded up to a multiple of 48, and also of 80 when M > 160 (the
   * 80-row tiles of the wide products). */
  int64_t frag_rows;
  /* the LayerNorm after O carried into FC1 (GATED_RES_LN / GELU_TANH_LN), optional:
   * ln_mean [max_rows] fp32 (the LN before QKV's row means), ln_stats [max_rows, D/16, 2] fp32,
   * ln_mod [16, D] bf16 */
  float* ln_mean;
  float* ln_stats;
  void* ln_mod;
} oasis_dit_buffers_t;

/* Conditioning for R frames: cond = MLP(timestep_embedding(t)) + ext(action) in fp32, then
 * ada[r, :] = silu(cond[r]) @ ada_w^T + ada_b for every sub-block (bf16 weights) and the final
 * layer (fp32 weights).
 *   t: fp32 [R]; action: fp32 [R, ext_dim_pad]; hid: fp32 [R, D] scratch; cond: fp32 [R, D];
 *   ada: fp32 [R, n_sub*6D + 2D].  R <= 1024.
 * (compute_cond_for_frame, oasis_inference.py:1406-1427; build_per_frame_adaln,
 * oasis_inference.py:971-993; silu_kernel call, oasis_inference.py:1459-1463.) */
int oasis_dit_conditioning(const oasis_dit_weights_t* w, const float* t, const float* action,
                           int64_t R, float* hid, float* cond, float* ada, oasis_stream_t stream);

/* oasis_dit_conditioning with no scratch argument, for callers that cannot allocate device
 * memory (code under hipGraph capture, tight serving loops, harnesses that forbid hipMalloc).
 * No counterpart in the reference. The MLP's hidden rows use a static device array of the
 * library (64 rows x 2048 columns of fp32, 512 KiB per GPU, held until the process ends), so
 * R <= 64 and d_model <= 2048 (larger: OASIS_ERR_SHAPE). Nothing is allocated; the first call on
 * a device looks up that device's copy of the array. Results equal oasis_dit_conditioning's
 * bit for bit. Calls that overlap on one GPU (concurrent streams or threads) share the array
 * and race; calls in sequence on one stream do not. */
int oasis_dit_conditioning_noalloc(const oasis_dit_weights_t* w, const float* t, const float* action,
                                   int64_t R, float* cond, float* ada, oasis_stream_t stream);

/* Sub-blocks [j0, j1) of the DiT on x[B*T*P, D] in place (j even: spatial, odd: temporal),
 * ada as in oasis_dit_forward.  (run_sub_block, oasis_inference.py:995-1215.) */
int oasis_dit_sub_blocks(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t B,
                         int64_t T, const float* ada, int64_t ada_fstride, int64_t j0, int64_t j1,
                         oasis_stream_t stream);

/* Final layer on x[M, D], fp32 throughout:
 * v_out[M, 64] = (LN(x) * scale_p1 + shift) @ final_w^T + final_b. (oasis_inference.py:1497-1521.) */
int oasis_dit_final(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t M,
                    const float* ada, int64_t ada_fstride, float* v_out, oasis_stream_t stream);

/* One DiT forward over B streams of T frames: x[B*T*P, D] holds the embedded tokens on
 * entry and the final hidden state on exit; v_out: fp32 [B*T*P, 64].
 * ada: adaLN rows, frame f = b*T + t at ada + f*ada_fstride.
 * (dit_forward_device, oasis_inference.py:1438-1526.) */
int oasis_dit_forward(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                      int64_t B, int64_t T, const float* ada, int64_t ada_fstride,
                      float* v_out, oasis_stream_t stream);

/* One full DiT denoising step for B streams of T frames (B*T <= 1024): conditioning MLP
 * (t fp32 [B*T], action fp32 [B*T, ext_dim_pad]), patch embed of patches fp32 [B*T*P, 64]
 * into buf->x, every sub-block and the final layer; v_out fp32 [B*T*P, 64].
 * hid/cond/ada: conditioning scratch as in oasis_dit_conditioning (B*T rows). The adaLN
 * rows of every consumer (the sub-blocks' bf16 stack and the final layer's fp32 rows) come
 * from one pass over the stacked adaLN weights before the first sub-block (one launch for up
 * to 8 conditioning rows).
 * (dit_forward_device with compute_cond_for_frame, oasis_inference.py:1406-1526.) */
int oasis_dit_step(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t B,
                   int64_t T, const float* t, const float* action, const float* patches,
                   float* hid, float* cond, float* ada, float* v_out, oasis_stream_t stream);

/* Temporal K/V cache of the context frame for the KV-cache DiT passes. For temporal
 * sub-block jt (sub-block j = 2*jt + 1), k + jt*S and v + jt*S (S = max_streams*P*2*D
 * elements) hold bf16 [max_streams][P][n_heads][2][64]: slot 0 the context (past) frame,
 * slot 1 the current frame. Caller-allocated, n_sub/2 * S elements each. */
typedef struct {
  void* k;
  void* v;
  int64_t max_streams;
} oasis_kv_cache_t;

/* Past-frame pass of the KV cache: buf->x [B*P, D] holds the B context frames' embedded
 * tokens; runs all sub-blocks at T=1 (temporal attention collapses to V) and stores every
 * temporal sub-block's rotated K and V in slot 0 of kv. No final layer; buf->x is left
 * holding the past frames' last hidden state. Needs buf->max_rows >= 2*B*P, w->t_max >= 2.
 * ada: the context frames' adaLN rows (stream b at ada + b*ada_fstride).
 * (precompute_past_state, oasis_inference.py:1354-1370, with run_sub_block_t1 in "save"
 * mode, oasis_inference.py:1218-1352.) */
int oasis_dit_precompute_past(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                              const oasis_kv_cache_t* kv, int64_t B, const float* ada,
                              int64_t ada_fstride, oasis_stream_t stream);

/* Current-frame pass of the KV cache: buf->x [B*P, D] holds the B current frames; runs all
 * sub-blocks at T=1, the temporal ones attending over [cached context K/V (slot 0), own K/V
 * (written to slot 1)], then the final layer: v_out fp32 [B*P, 64]. Equal to the current
 * rows of the T=2 forward (the context rows never see the current frame).
 * (dit_forward_currentonly, oasis_inference.py:1372-1403.) */
int oasis_dit_forward_current(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                              const oasis_kv_cache_t* kv, int64_t B, const float* ada,
                              int64_t ada_fstride, float* v_out, oasis_stream_t stream);

typedef struct {
  int depth;                 /* 12                                                 */
  int d_model;               /* 1024                                               */
  int n_heads;               /* 16                                                 */
  int d_mlp;                 /* 4096                                               */
  int latent_dim;            /* 32                                                 */
  int grid_h, grid_w;        /* 18 x 32                                            */
  int patch;                 /* 20                                                 */
  const void* pq_w;          /* [D, latent_dim]                                    */
  const float* pq_b;
  const float* n1_w[OASIS_MAX_SUB];
  const float* n1_b[OASIS_MAX_SUB];
  const void* qkv_w[OASIS_MAX_SUB];   /* [3D, D]                                   */
  const float* qkv_b[OASIS_MAX_SUB];
  const void* proj_w[OASIS_MAX_SUB];
  const float* proj_b[OASIS_MAX_SUB];
  const float* n2_w[OASIS_MAX_SUB];
  const float* n2_b[OASIS_MAX_SUB];
  const void* fc1_w[OASIS_MAX_SUB];
  const float* fc1_b[OASIS_MAX_SUB];
  const void* fc2_w[OASIS_MAX_SUB];
  const float* fc2_b[OASIS_MAX_SUB];
  const float* norm_w;
  const float* norm_b;
  const void* pred_w;        /* [3*patch*patch, D]                                 */
  const float* pred_b;
  const float* rope_cos;     /* [grid_h*grid_w, 64]                                */
  const float* rope_sinp;
} oasis_vae_weights_t;

/* Activation workspace for up to max_rows tokens (max_rows / L latents of L = grid_h*grid_w). */
typedef struct {
  int64_t max_rows;
  float* x;        /* [max_rows, D] fp32   */
  void* h;         /* [max_rows, D] bf16   */
  void* q;         /* [max_rows, D] bf16   */
  void* k;
  void* v;
  void* attn;      /* [max_rows, D] bf16   */
  void* mlp;       /* [max_rows, Dm] bf16  */
  float* partial;  /* [max_splits, max_rows, D] fp32 split-K slices */
  int64_t max_splits;
} oasis_vae_buffers_t;

/* latent fp32 [L, latent_dim] -> frame fp32 [3, grid_h*patch, grid_w*patch] in [-1, 1].
 * (vae_decode_forward, oasis_inference.py:1546-1618, + vae_unpatchify and clamp.) */
int oasis_vae_decode(const oasis_vae_weights_t* w, const oasis_vae_buffers_t* buf,
                     const float* latent, float* frame, oasis_stream_t stream);

/* B latents fp32 [B, L, latent_dim] -> B frames fp32 [B, 3, H, W], as one pass of B*L tokens
 * through every projection (attention stays within each latent); buf->max_rows >= B*L.
 * Results equal B calls of oasis_vae_decode up to the projections' summation order. (The
 * reference decodes one frame per vae_decode_forward call, oasis_inference.py:1546-1618; this
 * batches the decodes of several frames or streams.) */
int oasis_vae_decode_batch(const oasis_vae_weights_t* w, const oasis_vae_buffers_t* buf, int64_t B,
                           const float* latents, float* frames, oasis_stream_t stream);

/* B latents fp32 [B, L, latent_dim] -> the predictor's rows pred_out fp32 [B*L, ld_pred]
 * (ld_pred >= 3*patch^2; columns from 3*patch^2 on are not written): acc + bias, unclamped,
 * before any unpatchify. This is what the reference's vae_decode_forward returns
 * (vae_scr["pred_out"], oasis_inference.py:1546-1618) and vae_decode_device reads back
 * (oasis_inference.py:1620-1634) for the host-side vae_unpatchify. */
int oasis_vae_decode_patches(const oasis_vae_weights_t* w, const oasis_vae_buffers_t* buf, int64_t B,
                             const float* latents, float* pred_out, int64_t ld_pred, oasis_stream_t stream);

/* One generated frame at T=2: conditioning, n_steps DDIM v-prediction steps, then bridge +
 * VAE decode.
 *   chunk: fp32 [P, 64] noise in, denoised latent patches out;
 *   ctx_patches: fp32 [P, 64] context frame in patch space (embedded on device into ctx_z);
 *   t, action: fp32 [1 + n_steps] timesteps and [1 + n_steps, ext_dim_pad] actions; row 0 is
 *        the context frame, row 1 + i the generated frame at step i;
 *   coeffs: HOST array of n_steps x 6 DDIM coefficients (oasis_ddim_update order);
 *   hid/cond/ada: conditioning scratch as in oasis_dit_conditioning (1 + n_steps rows);
 *   ctx_z: fp32 [P, D] scratch; v_out: fp32 [2P, 64] scratch; latent: fp32 [4P, vae
 *   latent_dim] scratch; frame: fp32 [3, H, W] output. n_steps <= 15.
 * The adaLN projections of all conditioning rows run as one pass before the first step.
 * kv: NULL runs every step as the T=2 forward. Otherwise (a cache for >= 1 stream) step 0
 * runs at T=2 and stores the context frame's temporal K/V, and steps 1.. run only the
 * current frame at T=1 against that cache (the K/V-cache path of oasis_inference.py:
 * 1934-1963, with the past-frame pass folded into the first step).
 * (ddim_step_fn and the traced frame, oasis_inference.py:1909-1932,2131-2148.) */
int oasis_ddim_frame(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                     const oasis_vae_weights_t* vw, const oasis_vae_buffers_t* vbuf,
                     const oasis_kv_cache_t* kv, float* chunk, const float* ctx_patches, const float* t,
                     const float* action, int64_t n_steps, const float* coeffs, float* hid,
                     float* cond, float* ada, float* ctx_z, float* v_out, float* latent,
                     float* frame, oasis_stream_t stream);

/* n_frames consecutive generated frames of one stream with the context window rolled on
 * the device: frame f's context is frame f-1's denoised latent (frame 0: ctx_patches). Per
 * frame: context patch embed and n_steps DDIM steps (K/V cache as in oasis_ddim_frame). The
 * bridges + VAE decodes run after the last frame on `stream`, batched as oasis_video_decode
 * runs them. (To overlap the decodes with the next frames' DiT steps, run this with
 * frames = NULL on one stream and oasis_video_decode on another.)
 *   chunks: fp32 [n_frames, P, 64] noise in, denoised latents out;
 *   t, action: fp32 [n_frames * (1 + n_steps)] and [n_frames * (1 + n_steps), ext_dim_pad]:
 *        frame f's rows at f*(1 + n_steps), row 0 its context frame, row 1 + i step i;
 *   hid/cond/ada: conditioning scratch for n_frames * (1 + n_steps) rows;
 *   frames: fp32 [n_frames, 3, H, W], or NULL for the DiT half only (the chunks are the
 *        output; vbuf and latent may then be NULL; oasis_video_decode is the other half);
 *   latent: scratch as in oasis_video_decode;
 *   other arguments as in oasis_ddim_frame. n_frames <= 64.
 * The calls into one (w, buf) pair must not overlap. (The interactive loop's context roll,
 * oasis_inference.py:2296-2306, with play.py:241-531's per-frame DDIM + decode.) */
int oasis_video_frames(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                       const oasis_vae_weights_t* vw, const oasis_vae_buffers_t* vbuf,
                       const oasis_kv_cache_t* kv, int64_t n_frames, float* chunks,
                       const float* ctx_patches, const float* t, const float* action, int64_t n_steps,
                       const float* coeffs, float* hid, float* cond, float* ada, float* ctx_z,
                       float* v_out, float* latent, float* frames, oasis_stream_t stream);

/* The decode half of oasis_video_frames: for f < n_frames, the bridge of chunks[f] (denoised
 * latents fp32 [P, 64], (p,q,c) columns) into latent, then the VAE decode into frames[f] (fp32
 * [3, H, W], in [-1, 1]). The decodes run batched, as many latents per oasis_vae_decode_batch as
 * vbuf holds (vbuf->max_rows / 4P); latent is fp32 [that many, 4P, vae latent_dim] scratch. Run on
 * a second stream while the
 * next batch's oasis_video_frames(frames = NULL) runs on the first, the decodes overlap the
 * DiT steps. (bridge_unpatchify + vae_decode_forward + vae_unpatchify per frame,
 * oasis_inference.py:1651-1709,1546-1645; play.py:241-531's per-frame decode.) */
int oasis_video_decode(const oasis_dit_weights_t* w, const oasis_vae_weights_t* vw,
                       const oasis_vae_buffers_t* vbuf, int64_t n_frames, const float* chunks,
                       float* latent, float* frames, oasis_stream_t stream);

/* ---- hipGraph capture of any sequence of the calls above on one stream ---------
 * Replaces ttnn.begin_trace_capture / end_trace_capture / execute_trace / release_trace
 * (oasis_inference.py:2133-2146,2224; play.py:405-411). The stream must not be the
 * legacy default stream. */
int oasis_graph_begin(oasis_stream_t stream);
int oasis_graph_end(oasis_stream_t stream, void** graph_exec);
int oasis_graph_launch(void* graph_exec, oasis_stream_t stream);
int oasis_graph_destroy(void* graph_exec);

/* Blocks until all work queued on the stream is done (host helper for tests). */
int oasis_stream_sync(oasis_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* OASIS_HIP_H */
