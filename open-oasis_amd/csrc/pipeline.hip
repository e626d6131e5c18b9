// Composite entry points: conditioning, the DiT forward, the VAE decoder and one DDIM
// frame, each a fixed sequence of kernel launches on one stream (no allocation, no
// host synchronisation), plus hipGraph capture/replay of any such sequence and the
// library's error state.
#include <stdarg.h>
#include <stdio.h>

#include "oasis_common.h"

namespace oasis {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
}

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) {
    set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

}  // namespace oasis

#define OASIS_TRY(call)          \
  do {                           \
    const int _rc = (call);      \
    if (_rc != OASIS_OK) return _rc; \
  } while (0)

extern "C" const char* oasis_last_error(void) { return oasis::g_err; }
extern "C" int oasis_abi_version(void) { return OASIS_ABI_VERSION; }

namespace {

constexpr float kLnEps = 1e-6f;
constexpr float kAttnScale = 0.125f;  // 1/sqrt(64)

oasis_epilogue_t epi_zero() {
  oasis_epilogue_t e;
  memset(&e, 0, sizeof(e));
  return e;
}

int check_dit(const oasis_dit_weights_t* w) {
  OASIS_REQUIRE(w, OASIS_ERR_NULL, "dit: null weights");
  OASIS_REQUIRE(w->n_sub > 0 && w->n_sub <= OASIS_MAX_SUB && w->n_sub % 2 == 0, OASIS_ERR_SHAPE,
                "dit: n_sub=%d must be even and <= %d", w->n_sub, OASIS_MAX_SUB);
  OASIS_REQUIRE(w->n_heads > 0 && w->d_model == w->n_heads * 64, OASIS_ERR_SHAPE,
                "dit: d_model must be n_heads * 64");
  OASIS_REQUIRE(w->grid_h > 0 && w->grid_w > 0 && w->patch_dim == 64 && w->d_mlp > 0, OASIS_ERR_SHAPE,
                "dit: bad grid/patch/mlp dims");
  OASIS_REQUIRE(w->ada_w && w->ada_b && w->final_w && w->final_b && w->s_cos && w->s_sinp && w->t_cos &&
                    w->t_sinp,
                OASIS_ERR_NULL, "dit: missing weight pointer");
  for (int j = 0; j < w->n_sub; ++j)
    OASIS_REQUIRE(w->qkv_w[j] && w->out_w[j] && w->out_b[j] && w->fc1_w[j] && w->fc1_b[j] && w->fc2_w[j] &&
                      w->fc2_b[j],
                  OASIS_ERR_NULL, "dit: missing weights of sub-block %d", j);
  return OASIS_OK;
}

int64_t ada_width(const oasis_dit_weights_t* w) { return (int64_t)w->n_sub * 6 * w->d_model + 2 * w->d_model; }

}  // namespace

extern "C" int oasis_dit_conditioning(const oasis_dit_weights_t* w, const float* t, const float* action, int64_t R,
                                      float* tfreq, float* hid, float* cond, float* ada, oasis_stream_t stream) {
  OASIS_TRY(check_dit(w));
  OASIS_REQUIRE(t && action && tfreq && hid && cond && ada, OASIS_ERR_NULL, "dit_conditioning: null buffer");
  OASIS_REQUIRE(w->temb_w0 && w->temb_b0 && w->temb_w2 && w->temb_b2 && w->ext_w && w->ext_b, OASIS_ERR_NULL,
                "dit_conditioning: missing conditioning weights");
  const int64_t D = w->d_model, F = w->freq_dim, E = w->ext_dim_pad;
  OASIS_TRY(oasis_timestep_embedding(t, R, F, tfreq, stream));
  OASIS_TRY(oasis_gemv_bf16(tfreq, F, R, w->temb_w0, D, F, w->temb_b0, hid, D, OASIS_ACT_NONE, OASIS_ACT_SILU, 0,
                            stream));
  OASIS_TRY(oasis_gemv_bf16(action, E, R, w->ext_w, D, E, w->ext_b, cond, D, OASIS_ACT_NONE, OASIS_ACT_NONE, 0,
                            stream));
  OASIS_TRY(oasis_gemv_bf16(hid, D, R, w->temb_w2, D, D, w->temb_b2, cond, D, OASIS_ACT_NONE, OASIS_ACT_NONE, 1,
                            stream));
  const int64_t NA = ada_width(w);
  return oasis_gemv_bf16(cond, D, R, w->ada_w, NA, D, w->ada_b, ada, NA, OASIS_ACT_SILU, OASIS_ACT_NONE, 0, stream);
}

extern "C" int oasis_dit_sub_blocks(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t B,
                                    int64_t T, const float* ada, int64_t ada_fstride, int64_t j0, int64_t j1,
                                    oasis_stream_t stream) {
  OASIS_TRY(check_dit(w));
  OASIS_REQUIRE(buf && buf->x && buf->h && buf->q && buf->k && buf->v && buf->attn && buf->mlp, OASIS_ERR_NULL,
                "dit: missing buffer");
  OASIS_REQUIRE(ada, OASIS_ERR_NULL, "dit: null ada");
  OASIS_REQUIRE(B > 0 && T > 0 && T <= w->t_max, OASIS_ERR_SHAPE, "dit: need B > 0, 0 < T <= t_max (%d)", w->t_max);
  OASIS_REQUIRE(0 <= j0 && j0 <= j1 && j1 <= w->n_sub, OASIS_ERR_ARG, "dit: sub-block range [%lld, %lld) invalid",
                (long long)j0, (long long)j1);
  const int64_t D = w->d_model, H = w->n_heads, Dm = w->d_mlp;
  const int64_t P = (int64_t)w->grid_h * w->grid_w;
  const int64_t M = B * T * P;
  OASIS_REQUIRE(M <= buf->max_rows, OASIS_ERR_SHAPE, "dit: %lld rows exceed the workspace (%lld)", (long long)M,
                (long long)buf->max_rows);
  hipStream_t s = (hipStream_t)stream;

  oasis_epilogue_t qkv = epi_zero();
  qkv.kind = OASIS_EPI_QKV_ROPE;
  qkv.n_heads = (int)H;
  qkv.q = buf->q;
  qkv.k = buf->k;
  qkv.v = buf->v;
  qkv.rows_per_frame = P;
  qkv.frames_per_stream = T;

  oasis_epilogue_t gres = epi_zero();
  gres.kind = OASIS_EPI_GATED_RES;
  gres.out_f32 = buf->x;
  gres.ld_out = D;
  gres.gate_fstride = ada_fstride;
  gres.rows_per_frame = P;

  oasis_epilogue_t gelu = epi_zero();
  gelu.kind = OASIS_EPI_GELU_TANH;
  gelu.out_bf16 = buf->mlp;
  gelu.ld_out = Dm;

  // run_sub_block (oasis_inference.py:995-1215): sub-block j is spatial for even j
  for (int64_t j = j0; j < j1; ++j) {
    const bool spatial = (j % 2) == 0;
    const float* a = ada + j * 6 * D;  // shift_a, scale_a+1, gate_a, shift_m, scale_m+1, gate_m
    OASIS_TRY(oasis_ln_modulate(buf->x, M, D, a, a + D, ada_fstride, P, buf->h, kLnEps, stream));
    if (spatial) {  // heads-first per frame: [(b*T + t)*H + h][p][64]
      qkv.s_b = T * H * P * 64;
      qkv.s_t = H * P * 64;
      qkv.s_h = P * 64;
      qkv.s_p = 64;
      qkv.rope_cos = w->s_cos;
      qkv.rope_sinp = w->s_sinp;
      qkv.rope_by_frame = 0;
    } else {  // grouped by position: [b][p][h][t][64]
      qkv.s_b = P * H * T * 64;
      qkv.s_p = H * T * 64;
      qkv.s_h = T * 64;
      qkv.s_t = 64;
      qkv.rope_cos = w->t_cos;
      qkv.rope_sinp = w->t_sinp;
      qkv.rope_by_frame = 1;
    }
    OASIS_TRY(oasis::gemm_launch((const bf16*)buf->h, D, (const bf16*)w->qkv_w[j], D, M, 3 * D, D, qkv, s));
    if (spatial)
      OASIS_TRY(oasis_attention(buf->q, buf->k, buf->v, buf->attn, B * T, P, H, kAttnScale, stream));
    else
      OASIS_TRY(oasis_temporal_attention(buf->q, buf->k, buf->v, buf->attn, B, T, P, H, kAttnScale, stream));
    gres.bias = w->out_b[j];
    gres.gate = a + 2 * D;
    OASIS_TRY(oasis::gemm_launch((const bf16*)buf->attn, D, (const bf16*)w->out_w[j], D, M, D, D, gres, s));
    OASIS_TRY(oasis_ln_modulate(buf->x, M, D, a + 3 * D, a + 4 * D, ada_fstride, P, buf->h, kLnEps, stream));
    gelu.bias = w->fc1_b[j];
    OASIS_TRY(oasis::gemm_launch((const bf16*)buf->h, D, (const bf16*)w->fc1_w[j], D, M, Dm, D, gelu, s));
    gres.bias = w->fc2_b[j];
    gres.gate = a + 5 * D;
    OASIS_TRY(oasis::gemm_launch((const bf16*)buf->mlp, Dm, (const bf16*)w->fc2_w[j], Dm, M, D, Dm, gres, s));
  }
  return OASIS_OK;
}

extern "C" int oasis_dit_final(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t M,
                               const float* ada, int64_t ada_fstride, float* v_out, oasis_stream_t stream) {
  OASIS_TRY(check_dit(w));
  OASIS_REQUIRE(buf && buf->x && buf->h && ada && v_out, OASIS_ERR_NULL, "dit_final: null pointer");
  OASIS_REQUIRE(M > 0 && M <= buf->max_rows, OASIS_ERR_SHAPE, "dit_final: bad row count");
  const int64_t D = w->d_model, P = (int64_t)w->grid_h * w->grid_w;
  // final layer (oasis_inference.py:1497-1521): adaLN(2 chunks) + LN + modulate + linear
  const float* fa = ada + (int64_t)w->n_sub * 6 * D;
  OASIS_TRY(oasis_ln_modulate(buf->x, M, D, fa, fa + D, ada_fstride, P, buf->h, kLnEps, stream));
  oasis_epilogue_t fin = epi_zero();
  fin.kind = OASIS_EPI_STORE_F32;
  fin.bias = w->final_b;
  fin.out_f32 = v_out;
  fin.ld_out = w->patch_dim;
  return oasis::gemm_launch((const bf16*)buf->h, D, (const bf16*)w->final_w, D, M, w->patch_dim, D, fin,
                            (hipStream_t)stream);
}

extern "C" int oasis_dit_forward(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t B, int64_t T,
                                 const float* ada, int64_t ada_fstride, float* v_out, oasis_stream_t stream) {
  OASIS_REQUIRE(w, OASIS_ERR_NULL, "dit_forward: null weights");
  OASIS_TRY(oasis_dit_sub_blocks(w, buf, B, T, ada, ada_fstride, 0, w->n_sub, stream));
  return oasis_dit_final(w, buf, B * T * (int64_t)w->grid_h * w->grid_w, ada, ada_fstride, v_out, stream);
}

extern "C" int oasis_vae_decode(const oasis_vae_weights_t* w, const oasis_vae_buffers_t* buf, const float* latent,
                                float* frame, oasis_stream_t stream) {
  OASIS_REQUIRE(w && buf && latent && frame, OASIS_ERR_NULL, "vae_decode: null pointer");
  OASIS_REQUIRE(w->depth > 0 && w->depth <= OASIS_MAX_SUB && w->n_heads > 0 && w->d_model == w->n_heads * 64,
                OASIS_ERR_SHAPE, "vae_decode: bad depth/heads/d_model");
  OASIS_REQUIRE(buf->x && buf->h && buf->q && buf->k && buf->v && buf->attn && buf->mlp, OASIS_ERR_NULL,
                "vae_decode: missing buffer");
  OASIS_REQUIRE(w->pq_w && w->pq_b && w->norm_w && w->norm_b && w->pred_w && w->pred_b && w->rope_cos &&
                    w->rope_sinp,
                OASIS_ERR_NULL, "vae_decode: missing weight pointer");
  const int64_t D = w->d_model, H = w->n_heads, Dm = w->d_mlp;
  const int64_t L = (int64_t)w->grid_h * w->grid_w;
  hipStream_t s = (hipStream_t)stream;
  OASIS_TRY(oasis_small_linear(latent, w->latent_dim, L, w->latent_dim, w->pq_w, D, w->pq_b, buf->x, D, stream));

  oasis_epilogue_t qkv = epi_zero();
  qkv.kind = OASIS_EPI_QKV_ROPE;
  qkv.n_heads = (int)H;
  qkv.q = buf->q;
  qkv.k = buf->k;
  qkv.v = buf->v;
  qkv.rows_per_frame = L;
  qkv.frames_per_stream = 1;
  qkv.s_b = qkv.s_t = 0;
  qkv.s_h = L * 64;
  qkv.s_p = 64;
  qkv.rope_cos = w->rope_cos;
  qkv.rope_sinp = w->rope_sinp;
  oasis_epilogue_t res = epi_zero();
  res.kind = OASIS_EPI_RESIDUAL;
  res.out_f32 = buf->x;
  res.ld_out = D;
  oasis_epilogue_t gelu = epi_zero();
  gelu.kind = OASIS_EPI_GELU_ERF;
  gelu.out_bf16 = buf->mlp;
  gelu.ld_out = Dm;

  for (int i = 0; i < w->depth; ++i) {
    OASIS_REQUIRE(w->n1_w[i] && w->n1_b[i] && w->qkv_w[i] && w->qkv_b[i] && w->proj_w[i] && w->proj_b[i] &&
                      w->n2_w[i] && w->n2_b[i] && w->fc1_w[i] && w->fc1_b[i] && w->fc2_w[i] && w->fc2_b[i],
                  OASIS_ERR_NULL, "vae_decode: missing weights of block %d", i);
    OASIS_TRY(oasis_ln_affine(buf->x, L, D, w->n1_w[i], w->n1_b[i], buf->h, kLnEps, stream));
    qkv.bias = w->qkv_b[i];
    OASIS_TRY(oasis::gemm_launch((const bf16*)buf->h, D, (const bf16*)w->qkv_w[i], D, L, 3 * D, D, qkv, s));
    OASIS_TRY(oasis_attention(buf->q, buf->k, buf->v, buf->attn, 1, L, H, kAttnScale, stream));
    res.bias = w->proj_b[i];
    OASIS_TRY(oasis::gemm_launch((const bf16*)buf->attn, D, (const bf16*)w->proj_w[i], D, L, D, D, res, s));
    OASIS_TRY(oasis_ln_affine(buf->x, L, D, w->n2_w[i], w->n2_b[i], buf->h, kLnEps, stream));
    gelu.bias = w->fc1_b[i];
    OASIS_TRY(oasis::gemm_launch((const bf16*)buf->h, D, (const bf16*)w->fc1_w[i], D, L, Dm, D, gelu, s));
    res.bias = w->fc2_b[i];
    OASIS_TRY(oasis::gemm_launch((const bf16*)buf->mlp, Dm, (const bf16*)w->fc2_w[i], Dm, L, D, Dm, res, s));
  }
  OASIS_TRY(oasis_ln_affine(buf->x, L, D, w->norm_w, w->norm_b, buf->h, kLnEps, stream));
  oasis_epilogue_t pred = epi_zero();
  pred.kind = OASIS_EPI_UNPATCHIFY;
  pred.bias = w->pred_b;
  pred.out_f32 = frame;
  pred.rows_per_frame = L;
  pred.unpatch_grid_w = w->grid_w;
  pred.unpatch_patch = w->patch;
  pred.unpatch_channels = 3;
  return oasis::gemm_launch((const bf16*)buf->h, D, (const bf16*)w->pred_w, D, L,
                            3LL * w->patch * w->patch, D, pred, s);
}

extern "C" int oasis_ddim_frame(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                                const oasis_vae_weights_t* vw, const oasis_vae_buffers_t* vbuf, float* chunk,
                                const float* ctx_z, const float* ada, int64_t n_steps, const float* coeffs,
                                float* v_out, float* latent, float* frame, oasis_stream_t stream) {
  OASIS_TRY(check_dit(w));
  OASIS_REQUIRE(buf && vw && vbuf && chunk && ctx_z && ada && coeffs && v_out && latent && frame, OASIS_ERR_NULL,
                "ddim_frame: null pointer");
  OASIS_REQUIRE(n_steps > 0 && n_steps <= 1000, OASIS_ERR_ARG, "ddim_frame: bad step count");
  OASIS_REQUIRE(w->xemb_w && w->xemb_b, OASIS_ERR_NULL, "ddim_frame: missing patch-embed weights");
  const int64_t D = w->d_model, P = (int64_t)w->grid_h * w->grid_w, C = w->patch_dim / 4;
  OASIS_REQUIRE(2 * P <= buf->max_rows, OASIS_ERR_SHAPE, "ddim_frame: workspace too small for T=2");
  OASIS_REQUIRE((int64_t)vw->grid_h * vw->grid_w == 4 * P && vw->latent_dim >= C, OASIS_ERR_SHAPE,
                "ddim_frame: VAE grid must be the 2x-upsampled DiT grid");
  const int64_t NA = ada_width(w);
  hipStream_t s = (hipStream_t)stream;
  for (int64_t i = 0; i < n_steps; ++i) {
    if (hipMemcpyAsync(buf->x, ctx_z, P * D * sizeof(float), hipMemcpyDeviceToDevice, s) != hipSuccess)
      return oasis::check_launch("ddim_frame context copy");
    OASIS_TRY(oasis_small_linear(chunk, w->patch_dim, P, w->patch_dim, w->xemb_w, D, w->xemb_b, buf->x + P * D, D,
                                 stream));
    OASIS_TRY(oasis_dit_forward(w, buf, 1, 2, ada, (1 + i) * NA, v_out, stream));
    const float* c = coeffs + 6 * i;
    OASIS_TRY(oasis_ddim_update(chunk, v_out + P * w->patch_dim, P * w->patch_dim, c[0], c[1], c[2], c[3], c[4], c[5],
                                stream));
  }
  OASIS_TRY(oasis_bridge(chunk, latent, w->grid_h, w->grid_w, C, vw->latent_dim, 1.0f / 0.07843137255f, stream));
  return oasis_vae_decode(vw, vbuf, latent, frame, stream);
}

extern "C" int oasis_graph_begin(oasis_stream_t stream) {
  OASIS_REQUIRE(stream, OASIS_ERR_ARG, "graph_begin: capture needs a non-default stream");
  const hipError_t e = hipStreamBeginCapture((hipStream_t)stream, hipStreamCaptureModeThreadLocal);
  if (e != hipSuccess) {
    oasis::set_error("hipStreamBeginCapture failed: %s", hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

extern "C" int oasis_graph_end(oasis_stream_t stream, void** graph_exec) {
  OASIS_REQUIRE(stream && graph_exec, OASIS_ERR_NULL, "graph_end: null argument");
  hipGraph_t g = nullptr;
  hipError_t e = hipStreamEndCapture((hipStream_t)stream, &g);
  if (e != hipSuccess) {
    oasis::set_error("hipStreamEndCapture failed: %s", hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  hipGraphExec_t x = nullptr;
  e = hipGraphInstantiate(&x, g, nullptr, nullptr, 0);
  (void)hipGraphDestroy(g);
  if (e != hipSuccess) {
    oasis::set_error("hipGraphInstantiate failed: %s", hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  *graph_exec = x;
  return OASIS_OK;
}

extern "C" int oasis_graph_launch(void* graph_exec, oasis_stream_t stream) {
  OASIS_REQUIRE(graph_exec, OASIS_ERR_NULL, "graph_launch: null graph");
  const hipError_t e = hipGraphLaunch((hipGraphExec_t)graph_exec, (hipStream_t)stream);
  if (e != hipSuccess) {
    oasis::set_error("hipGraphLaunch failed: %s", hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

extern "C" int oasis_graph_destroy(void* graph_exec) {
  if (!graph_exec) return OASIS_OK;
  const hipError_t e = hipGraphExecDestroy((hipGraphExec_t)graph_exec);
  if (e != hipSuccess) {
    oasis::set_error("hipGraphExecDestroy failed: %s", hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

extern "C" int oasis_stream_sync(oasis_stream_t stream) {
  const hipError_t e = hipStreamSynchronize((hipStream_t)stream);
  if (e != hipSuccess) {
    oasis::set_error("hipStreamSynchronize failed: %s", hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}
