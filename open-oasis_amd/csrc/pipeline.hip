// Composite entry points: conditioning, the DiT forward, the VAE decoder and one DDIM
// frame, each a fixed sequence of kernel launches on one stream (no allocation, no
// host synchronisation), plus hipGraph capture/replay of any such sequence and the
// library's error state.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>

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

#include <stdlib.h>

#include <mutex>
#include <string>

namespace {

// GEMM plan per projection role: tile configuration (-1 = gemm.hip's default for the
// shape) and split-K count (0 = chosen from the shape). Tuning override, read once (the only
// process-wide state besides the per-thread error text and the per-device address of the
// not-allocating entry point's scratch):
//   OASIS_GEMM_PLAN="qkv:1,o:0:4,fc1:2,fc2:2:4,vqkv:3,vo:2:2,vfc1:4,vfc2:2:2" (tile ids of gemm.hip)
enum { ROLE_QKV, ROLE_O, ROLE_FC1, ROLE_FC2, ROLE_VQKV, ROLE_VO, ROLE_VFC1, ROLE_VFC2, ROLE_N };
struct Plan {
  int tile[ROLE_N];
  int splits[ROLE_N];
  int tile8[ROLE_N];  // fp8-weight tiles (kTiles8 ids of gemm_fp8.hip; OASIS_GEMM_PLAN8="fc1:10,...")
  // two-frame temporal windows on temporal_qkv.hip (OASIS_TEMPORAL_FUSED): 0 for none (default:
  // the wave-split QKV GEMM + temporal attention pair times as fast or faster on MI355X, 1.592
  // against 1.601 ms per step and 160.9 against 160.6 FPS per frame), 1 for the T = 2 passes,
  // 2 for every pass
  int fused_temporal;
  // which operands are kept in MFMA fragment order, with their projection on gemm_frag: a mask of
  // the FRAG_* bits for passes of at most 160 tokens (frag1) and of 161 to 320 (frag2). OASIS_FRAG
  // = "frag1[,frag2]" (0 for none). The defaults, O and FC2 with the carried LayerNorm at both
  // sizes, are the fastest masks measured on MI355X with the weights read ahead (pf_host): the T = 2
  // step 1.4470 ms against 1.4644 without FC2 at two frames; the QKV bit changes nothing.
  int frag1, frag2;
  // weights read ahead into the memory-side cache by extra workgroups of the kernels before the
  // projections, in the DiT's passes of at most 320 tokens (bf16 weights): for the QKV, O, FC1 and
  // FC2 weights, which kernel of a sub-block reads them (PF_NONE; PF_LN, the residual + LN at its
  // start, and PF_ATTN, its attention, in a second grid slice; PF_QKVG, PF_OG, PF_FC1G and PF_FC2G,
  // the QKV, O, FC1 and FC2 GEMMs' workgroups past their tiles, on the CUs the tiles leave idle).
  // A host that runs at or after a weight's projection reads the next sub-block's copy of it.
  // OASIS_PREFETCH = "qkv,o,fc1,fc2" codes for both pass sizes, or eight for up to 160 tokens and
  // for 161 to 320. A CU issues these one-word reads slowly, so each host takes what its idle CUs
  // read in its own time. The defaults are the fastest placements measured on MI355X (one box, two
  // reps each):
  //  - two frames (256 tiles in FC1 and FC2, none idle): QKV's during the LN, O's during the QKV
  //    GEMM (16 idle CUs), FC1's during O (64), FC2's during the attention: the T = 2 step 1.4250
  //    ms, against 1.4383 with FC1's during the attention too, 1.4580 with FC1's and FC2's during
  //    O, 1.4846 with none, and 1.61-1.86 ms with FC1's or FC2's on the QKV GEMM's 16 idle CUs;
  //  - one frame (FC1 and FC2 leave 64 CUs idle): the next sub-block's QKV and this one's FC2
  //    during FC1, O's during QKV, FC1's during O: the K/V-cache frame 5.486 ms, against 5.602
  //    with the two-frame placement and 5.534 with only FC2's moved to FC1.
  int pf_host[2][4];  // passes of up to 160 tokens, of 161 to 320
  // log2 of the bytes between the words read, for DiT passes of up to 160 tokens, of 161 to 320,
  // and the VAE (OASIS_PF_LINE = "a,b,c", 4 to 8). A word every 128 bytes does not bring every
  // byte into the cache: a word every 64 takes the K/V-cache frame from 5.731 to 5.656 ms, the
  // one-frame passes having idle CUs to spare, and leaves the T = 2 step and the VAE unchanged;
  // a word every 256 bytes is slower than none (step 1.4876, frame 5.952 ms), and every 32 or 16
  // bytes slower again (frame 5.68 and 6.02 ms).
  int pf_line[3];
  // Large-token passes whose unsplit 144 x 128 tiles fill the 256 CUs (4465+ tokens at D = 1024):
  // the O and FC2 projections (N = D) unsplit on these tiles (bf16 kTiles id, fp8 kTiles8 id) with
  // the bias + gated residual into x in their epilogue, so that no split-K partials are written and
  // read back and the LayerNorm + modulate after them runs alone. OASIS_O_UNSPLIT and
  // OASIS_FC2_UNSPLIT = "bf16_tile,fp8_tile" (-1: split-K partials + residual_ln). The defaults
  // are the fastest measured on MI355X (one box, two reps each), against split-K on 288 x 128:
  //  - bf16 tile 16 (144 x 128, 6 waves, 4 stages), fp8 tile 10 (the same, 3 stages): the config-2
  //    sub-block 0.204 -> 0.188 ms, the config-4 step 6.31 -> 5.91 ms (bf16) and 5.61 -> 5.22 ms (fp8);
  //  - two stages (bf16 tile 13, fp8 8): 6.59 / 5.65 ms with FC2 unsplit; O alone 6.22 / 5.44 ms;
  //  - 8 waves of 144 x 16 on 288 x 64 (bf16 14, fp8 9): O alone 6.53 / 5.65 ms;
  //  - FC1 or QKV on the 144 x 128 tiles too (four rounds of 256 tiles): 6.52-7.04 / 5.52-5.99 ms.
  int o_unsplit[2];
  int fc2_unsplit[2];
};

enum { PF_NONE = 0, PF_LN = 1, PF_ATTN = 2, PF_QKVG = 3, PF_OG = 4, PF_FC1G = 5, PF_FC2G = 6 };
// where each host runs in a sub-block, and where each of the four weights is read: a host that runs
// at or after a weight's projection reads the next sub-block's copy of it
constexpr int kHostPos[7] = {-1, 0, 2, 1, 3, 4, 5};
constexpr int kWeightPos[4] = {1, 3, 4, 5};  // QKV, O, FC1, FC2
// the VAE decoder's blocks (decodes of fewer than 2048 tokens): QKV's weights during the LN before
// it, O's, FC1's and FC2's during the attention
constexpr int kVaePrefetch[4] = {PF_LN, PF_ATTN, PF_ATTN, PF_ATTN};

// Fragment-order operands, one bit each: the LN output QKV reads, the attention output O reads,
// the LN output FC1 reads, and FC1's GELU output FC2 reads. FRAG_LN (with FRAG_O) carries the
// LayerNorm + modulate after O into FC1 (GATED_RES_LN / GELU_TANH_LN): one residual_ln launch
// fewer per sub-block, FC1 on gemm_frag whatever FRAG_FC1 says.
enum { FRAG_QKV = 1, FRAG_O = 2, FRAG_FC1 = 4, FRAG_FC2 = 8, FRAG_LN = 16, FRAG_ALL = 31 };

const Plan& plan() {
  static Plan p = [] {
    Plan q;
    for (int i = 0; i < ROLE_N; ++i) {
      q.tile[i] = -1;
      q.splits[i] = 0;
    }
    q.fused_temporal = 0;
    static const char* names[ROLE_N] = {"qkv", "o", "fc1", "fc2", "vqkv", "vo", "vfc1", "vfc2"};
    if (const char* env = getenv("OASIS_GEMM_PLAN")) {
      std::string str(env);
      size_t pos = 0;
      while (pos < str.size()) {
        size_t end = str.find(',', pos);
        if (end == std::string::npos) end = str.size();
        const std::string item = str.substr(pos, end - pos);
        pos = end + 1;
        const size_t c1 = item.find(':');
        if (c1 == std::string::npos) continue;
        const std::string name = item.substr(0, c1);
        int tile = -1, splits = 0;
        if (sscanf(item.c_str() + c1 + 1, "%d:%d", &tile, &splits) < 1) continue;
        for (int i = 0; i < ROLE_N; ++i)
          if (name == names[i]) {
            q.tile[i] = tile;
            q.splits[i] = splits;
          }
      }
    }
    for (int i = 0; i < ROLE_N; ++i) q.tile8[i] = -1;
    if (const char* env = getenv("OASIS_GEMM_PLAN8")) {
      std::string str(env);
      size_t pos = 0;
      while (pos < str.size()) {
        size_t end = str.find(',', pos);
        if (end == std::string::npos) end = str.size();
        const std::string item = str.substr(pos, end - pos);
        pos = end + 1;
        const size_t c1 = item.find(':');
        int tile = -1;
        if (c1 == std::string::npos || sscanf(item.c_str() + c1 + 1, "%d", &tile) < 1) continue;
        for (int i = 0; i < ROLE_N; ++i)
          if (item.substr(0, c1) == names[i]) q.tile8[i] = tile;
      }
    }
    if (const char* env = getenv("OASIS_TEMPORAL_FUSED")) q.fused_temporal = atoi(env);
    // one frame: the next sub-block's QKV and this one's FC2 during FC1, O's during QKV, FC1's
    // during O; two frames: QKV's during the LN, O's during QKV, FC1's during O, FC2's during the
    // attention
    const int pf1[4] = {PF_FC1G, PF_QKVG, PF_OG, PF_FC1G}, pf2[4] = {PF_LN, PF_QKVG, PF_OG, PF_ATTN};
    for (int r = 0; r < 4; ++r) {
      q.pf_host[0][r] = pf1[r];
      q.pf_host[1][r] = pf2[r];
    }
    q.pf_line[0] = 6;
    q.pf_line[1] = q.pf_line[2] = 7;
    if (const char* env = getenv("OASIS_PF_LINE")) {
      int l[3] = {0, 0, 0};
      sscanf(env, "%d,%d,%d", &l[0], &l[1], &l[2]);
      for (int i = 0; i < 3; ++i)
        if (l[i] >= 4 && l[i] <= 8) q.pf_line[i] = l[i];
    }
    if (const char* env = getenv("OASIS_PREFETCH")) {
      int h[8] = {0, 0, 0, 0, 0, 0, 0, 0};
      const int n = sscanf(env, "%d,%d,%d,%d,%d,%d,%d,%d", &h[0], &h[1], &h[2], &h[3], &h[4], &h[5], &h[6], &h[7]);
      for (int i = 0; i < 8; ++i) {
        const int v = n > 4 ? h[i] : h[i % 4];  // four codes: both pass sizes
        q.pf_host[i / 4][i % 4] = (v >= PF_LN && v <= PF_FC2G) ? v : PF_NONE;
      }
    }
    q.o_unsplit[0] = q.fc2_unsplit[0] = 16;
    q.o_unsplit[1] = q.fc2_unsplit[1] = 10;
    if (const char* env = getenv("OASIS_O_UNSPLIT")) sscanf(env, "%d,%d", &q.o_unsplit[0], &q.o_unsplit[1]);
    if (const char* env = getenv("OASIS_FC2_UNSPLIT")) sscanf(env, "%d,%d", &q.fc2_unsplit[0], &q.fc2_unsplit[1]);
    q.frag1 = FRAG_O | FRAG_FC2 | FRAG_LN;
    q.frag2 = FRAG_O | FRAG_FC2 | FRAG_LN;
    if (const char* env = getenv("OASIS_FRAG")) {
      int a = 0, b = 0;
      const int n = sscanf(env, "%d,%d", &a, &b);
      if (n >= 1) q.frag1 = q.frag2 = a & FRAG_ALL;
      if (n == 2) q.frag2 = b & FRAG_ALL;
    }
    return q;
  }();
  return p;
}

}  // namespace

#define OASIS_TRY(call)          \
  do {                           \
    const int _rc = (call);      \
    if (_rc != OASIS_OK) return _rc; \
  } while (0)

extern "C" const char* oasis_last_error(void) { return oasis::g_err; }
extern "C" int oasis_abi_version(void) { return OASIS_ABI_VERSION; }

extern "C" int oasis_dit_frag_plan(int64_t rows) {
  if (rows <= 0 || rows > 320) return 0;
  return rows <= 160 ? plan().frag1 : plan().frag2;
}

extern "C" int64_t oasis_abi_struct_size(int which) {
  switch (which) {
    case 0: return sizeof(oasis_epilogue_t);
    case 1: return sizeof(oasis_dit_weights_t);
    case 2: return sizeof(oasis_dit_buffers_t);
    case 3: return sizeof(oasis_vae_weights_t);
    case 4: return sizeof(oasis_vae_buffers_t);
    default: return -1;
  }
}

namespace {

constexpr float kLnEps = 1e-6f;
constexpr float kAttnScale = 0.125f;  // 1/sqrt(64)
constexpr float kInvScaling = 1.0f / 0.07843137255f;  // 1 / scaling_factor (oasis_inference.py:107)

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
  OASIS_REQUIRE(w->ada_w && w->ada_b && w->final_ada_w && w->final_ada_b && w->final_w && w->final_b && w->s_cos &&
                    w->s_sinp && w->t_cos && w->t_sinp,
                OASIS_ERR_NULL, "dit: missing weight pointer");
  for (int j = 0; j < w->n_sub; ++j)
    OASIS_REQUIRE(w->qkv_w[j] && w->out_w[j] && w->out_b[j] && w->fc1_w[j] && w->fc1_b[j] && w->fc2_w[j] &&
                      w->fc2_b[j],
                  OASIS_ERR_NULL, "dit: missing weights of sub-block %d", j);
  OASIS_REQUIRE(w->weight_format == OASIS_WEIGHTS_BF16 || w->weight_format == OASIS_WEIGHTS_FP8, OASIS_ERR_ARG,
                "dit: unknown weight_format %d", w->weight_format);
  if (w->weight_format == OASIS_WEIGHTS_FP8) {
    OASIS_REQUIRE(w->d_model % 128 == 0 && w->d_mlp % 128 == 0, OASIS_ERR_SHAPE,
                  "dit: fp8 weights need d_model and d_mlp multiples of 128");
    for (int j = 0; j < w->n_sub; ++j)
      OASIS_REQUIRE(w->qkv_s[j] && w->out_s[j] && w->fc1_s[j] && w->fc2_s[j], OASIS_ERR_NULL,
                    "dit: missing fp8 scales of sub-block %d", j);
  }
  return OASIS_OK;
}

// One projection of sub-block j (role QKV/O/FC1/FC2): the bf16 GEMM on a bf16 A, or,
// with e4m3 weights, the fp8 GEMM on A given as fp8 blocks (A e4m3 bytes, A_scale e8m0).
int proj(const oasis_dit_weights_t* w, int role, int64_t j, const void* A, int64_t lda, const void* A_scale,
         int64_t M, int64_t N, int64_t K, const oasis_epilogue_t& e, int tile, int splits, hipStream_t s,
         const oasis::Prefetch* pf = nullptr, int tile8 = -1) {
  const void* W = role == ROLE_QKV ? w->qkv_w[j] : role == ROLE_O ? w->out_w[j] : role == ROLE_FC1 ? w->fc1_w[j]
                                                                                                   : w->fc2_w[j];
  if (w->weight_format == OASIS_WEIGHTS_FP8) {
    const float* sc = role == ROLE_QKV ? w->qkv_s[j] : role == ROLE_O ? w->out_s[j] : role == ROLE_FC1 ? w->fc1_s[j]
                                                                                                       : w->fc2_s[j];
    return oasis::gemm_fp8_launch(A, lda, (const uint8_t*)A_scale, K / 32, (const uint8_t*)W, K, sc, M, N, K, e,
                                  tile8 >= 0 ? tile8 : plan().tile8[role], splits, s);
  }
  return oasis::gemm_launch_cfg((const bf16*)A, lda, (const bf16*)W, K, M, N, K, e, tile, splits, s, pf);
}

// the prefetch ranges of one host kernel (PF_LN or PF_ATTN): the weights of the block's QKV, O,
// FC1 and FC2 (bytes[r] of each) that the plan assigns to it
oasis::Prefetch prefetch_for(const int (&hosts)[4], int host, bool on, const void* const (&wp)[4],
                             const int64_t (&bytes)[4], int line_log2, const void* const* wp_next = nullptr) {
  oasis::Prefetch pf = {{nullptr, nullptr, nullptr, nullptr}, {0, 0, 0, 0}, line_log2};
  if (!on) return pf;
  for (int r = 0; r < 4; ++r) {
    if (hosts[r] != host) continue;
    const void* p = kHostPos[host] < kWeightPos[r] ? wp[r] : (wp_next ? wp_next[r] : nullptr);
    if (p) oasis::prefetch_add(pf, p, bytes[r]);
  }
  return pf;
}

int64_t ada_width(const oasis_dit_weights_t* w) { return (int64_t)w->n_sub * 6 * w->d_model + 2 * w->d_model; }

}  // namespace

namespace {

// conditioning MLP for R rows in fp32: cond = W2 silu(W0 temb(t) + b0) + b2 + Wext action + bext
// (compute_cond_for_frame, oasis_inference.py:1406-1427) in two launches: the embedding is
// formed inside the first GEMV, and the second multiplies [hid | action] by [W2 | Wext]
int cond_mlp(const oasis_dit_weights_t* w, const float* t, const float* action, int64_t R, float* hid, float* cond,
             oasis_stream_t stream) {
  OASIS_REQUIRE(t && action && hid && cond, OASIS_ERR_NULL, "conditioning: null buffer");
  OASIS_REQUIRE(w->temb_w0 && w->temb_b0 && w->cond_w && w->cond_b, OASIS_ERR_NULL,
                "conditioning: missing conditioning weights");
  const int64_t D = w->d_model, F = w->freq_dim, E = w->ext_dim_pad;
  OASIS_TRY(oasis_gemv_f32(t, 1, R, w->temb_w0, D, F, w->temb_b0, hid, D, OASIS_ACT_TEMB, OASIS_ACT_SILU, 0, stream));
  return oasis::gemv_f32_cat(hid, D, D, action, E, R, w->cond_w, D, D + E, w->cond_b, cond, D, OASIS_ACT_NONE,
                             OASIS_ACT_NONE, 0, (hipStream_t)stream);
}

// adaLN rows of R conditioning rows: the sub-blocks' (bf16 weights) in one pass, then the
// final layer's (fp32 weights) at column n_sub*6D
int adaln_rows(const oasis_dit_weights_t* w, const float* cond, int64_t R, float* ada, hipStream_t s) {
  const int64_t D = w->d_model, NA = ada_width(w), NS = (int64_t)w->n_sub * 6 * D;
  // up to 8 rows (a step, a frame): one launch for both
  const int pair = oasis::gemv_adaln_pair(cond, D, R, w->ada_w, NS, w->ada_b, ada, w->final_ada_w, 2 * D,
                                          w->final_ada_b, ada + NS, D, NA, s);
  if (pair != 1) return pair;
  OASIS_TRY(oasis_gemv_bf16_tiled(cond, D, R, w->ada_w, NS, D, w->ada_b, ada, NA, OASIS_ACT_SILU, OASIS_ACT_NONE, 0,
                                  s));
  return oasis_gemv_f32(cond, D, R, w->final_ada_w, 2 * D, D, w->final_ada_b, ada + NS, NA, OASIS_ACT_SILU,
                        OASIS_ACT_NONE, 0, s);
}

}  // namespace

extern "C" int oasis_dit_conditioning(const oasis_dit_weights_t* w, const float* t, const float* action, int64_t R,
                                      float* hid, float* cond, float* ada, oasis_stream_t stream) {
  OASIS_TRY(check_dit(w));
  OASIS_REQUIRE(t && action && hid && cond && ada, OASIS_ERR_NULL, "dit_conditioning: null buffer");
  OASIS_TRY(cond_mlp(w, t, action, R, hid, cond, stream));
  return adaln_rows(w, cond, R, ada, (hipStream_t)stream);
}

// ---- oasis_dit_conditioning without a caller-supplied scratch buffer -------------------
// The MLP's hidden rows live in `scratch`, a file-scope device array: each GPU the library
// runs on holds its own copy (512 KiB) until the process ends. Host code never passes the
// array's name to a kernel (on the host it is a stand-in, not a device address): the first
// call on a device looks up that device's address with hipGetSymbolAddress and keeps it.
namespace {

constexpr int64_t kScratchRows = 64;    // conditioning rows per call
constexpr int64_t kScratchCols = 2048;  // d_model
static __device__ __align__(256) float scratch[kScratchRows * kScratchCols];

int scratch_ptr(float** out) {
  static std::mutex mu;
  static float* table[64] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    oasis::set_error("dit_conditioning_noalloc: no current device");
    return OASIS_ERR_LAUNCH;
  }
  std::lock_guard<std::mutex> lock(mu);
  if (!table[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      oasis::set_error("dit_conditioning_noalloc: hipGetSymbolAddress failed: %s", hipGetErrorString(e));
      return OASIS_ERR_LAUNCH;
    }
    table[dev] = static_cast<float*>(p);
  }
  *out = table[dev];
  return OASIS_OK;
}

}  // namespace

extern "C" int oasis_dit_conditioning_noalloc(const oasis_dit_weights_t* w, const float* t, const float* action,
                                              int64_t R, float* cond, float* ada, oasis_stream_t stream) {
  OASIS_TRY(check_dit(w));
  OASIS_REQUIRE(t && action && cond && ada, OASIS_ERR_NULL, "dit_conditioning_noalloc: null buffer");
  OASIS_REQUIRE(R > 0 && R <= kScratchRows, OASIS_ERR_SHAPE,
                "dit_conditioning_noalloc: R=%lld exceeds the %lld rows of its static scratch (use "
                "oasis_dit_conditioning)", (long long)R, (long long)kScratchRows);
  OASIS_REQUIRE(w->d_model <= kScratchCols, OASIS_ERR_SHAPE,
                "dit_conditioning_noalloc: d_model=%d exceeds the static scratch's %lld columns", w->d_model,
                (long long)kScratchCols);
  float* hid = nullptr;
  OASIS_TRY(scratch_ptr(&hid));
  // every row of hid that the second GEMV reads is written by the first one: nothing to clear
  OASIS_TRY(cond_mlp(w, t, action, R, hid, cond, stream));
  return adaln_rows(w, cond, R, ada, (hipStream_t)stream);
}

namespace {

// Split-K count of a partial-sum projection (O: K = D, FC2: K = 4D) below 2048 tokens, from timings
// on MI355X of gemm.hip's default tiles: O in 2 slices at one 144-token frame and whole above (the
// wave-split tiles fill the CUs without slicing), FC2 in 4; fewer when max_splits or whole 64-wide K
// tiles per slice require it. From 2048 tokens up the GEMM's own large-token tiles decide.
int choose_splits(int64_t M, int64_t N, int64_t K, int64_t max_splits) {
  (void)N;
  if (M >= 2048) return oasis::gemm_auto_splits(M, N, K, (int)std::min<int64_t>(max_splits, 8));
  int s = K > 1024 ? 4 : (M <= 160 ? 2 : 1);
  while (s > 1 && (s > max_splits || (K / 64) % s != 0)) s /= 2;
  return s;
}

// A residual that has been computed as split-K partials but not yet added to x.
struct Pending {
  const float* bias = nullptr;
  const float* gate = nullptr;
  int n = 0;
};

// x[m, :] += acc + bias: a projection's residual in its epilogue
oasis_epilogue_t residual_epi(float* x, int64_t ld, const float* bias) {
  oasis_epilogue_t e = epi_zero();
  e.kind = OASIS_EPI_RESIDUAL;
  e.bias = bias;
  e.out_f32 = x;
  e.ld_out = ld;
  return e;
}

// x[m, :] += gate[m / rows_per_frame, :] * (acc + bias): a projection's gated residual in its epilogue
oasis_epilogue_t gated_res_epi(float* x, int64_t ld, const float* bias, const float* gate, int64_t gate_fstride,
                               int64_t rows_per_frame) {
  oasis_epilogue_t e = epi_zero();
  e.kind = OASIS_EPI_GATED_RES;
  e.bias = bias;
  e.out_f32 = x;
  e.ld_out = ld;
  e.gate = gate;
  e.gate_fstride = gate_fstride;
  e.rows_per_frame = rows_per_frame;
  return e;
}

oasis_epilogue_t partial_epi(float* part, int64_t M, int64_t N) {
  oasis_epilogue_t e = epi_zero();
  e.kind = OASIS_EPI_PARTIAL_F32;
  e.out_f32 = part;
  e.ld_out = N;
  e.split_stride = M * N;
  return e;
}

int check_dit_buf(const oasis_dit_buffers_t* buf, const oasis_dit_weights_t* w) {
  OASIS_REQUIRE(buf && buf->x && buf->h && buf->q && buf->k && buf->v && buf->attn && buf->mlp && buf->partial,
                OASIS_ERR_NULL, "dit: missing buffer");
  OASIS_REQUIRE(buf->max_splits >= 1, OASIS_ERR_ARG, "dit: max_splits must be >= 1");
  OASIS_REQUIRE(w->weight_format != OASIS_WEIGHTS_FP8 ||
                    (buf->act8 && buf->act8_scale && buf->mlp8 && buf->mlp8_scale),
                OASIS_ERR_NULL, "dit: fp8 weights need the act8/mlp8 buffers");
  return OASIS_OK;
}

// How a forward pass uses the temporal K/V cache (oasis_kv_cache_t): SAVE_T2 is a T=2
// pass whose temporal K/V go to the cache (context in slot 0, current in slot 1);
// SAVE_T1 a T=1 pass over the context frames (slot 0, attention output = V); USE_T1 a T=1
// pass over the current frames (slot 1) attending over both slots.
enum { KV_NONE, KV_SAVE_T2, KV_SAVE_T1, KV_USE_T1 };
struct KvPass {
  bf16* k = nullptr;
  bf16* v = nullptr;
  int64_t sub_stride = 0;  // elements per temporal sub-block
  int mode = KV_NONE;
};

// The FRAG_* operands a pass of M tokens over sub-blocks [j0, j1) keeps in fragment order: the
// plan's mask for its size, narrowed to the roles whose fragment-order weights every sub-block has.
// None without bf16 weights, past 320 tokens or whole 48-row tiles, without the rounded-up rows in
// the buffers, with a per-role tile override or the fused temporal kernel (those read row-major
// operands), or at a model width the kernel's K slices do not cover (D <= 1024; FC2 in slices of
// 1024 or less).
int frag_mask(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t M, int64_t j0, int64_t j1,
              int fc2_splits) {
  const Plan& pl = plan();
  int m = M <= 160 ? pl.frag1 : pl.frag2;
  if (!m || pl.fused_temporal > 0 || w->weight_format != OASIS_WEIGHTS_BF16) return 0;
  for (int r = 0; r < ROLE_N; ++r)
    if (pl.tile[r] >= 0 || pl.splits[r] > 0) return 0;
  const int64_t D = w->d_model, Dm = w->d_mlp;
  if (M > 320 || M % 48 != 0 || buf->frag_rows < oasis::gemm_frag_rows(M)) return 0;
  if (!(D == 256 || D == 512 || D == 1024)) return 0;
  const int64_t sl = fc2_splits >= 1 && Dm % fc2_splits == 0 ? Dm / fc2_splits : 0;
  if (!(sl == 256 || sl == 512 || sl == 1024)) m &= ~FRAG_FC2;
  for (int64_t j = j0; j < j1; ++j) {
    if (!w->qkv_wf[j]) m &= ~FRAG_QKV;
    if (!w->out_wf[j]) m &= ~FRAG_O;
    if (!w->fc1_wf[j]) m &= ~(FRAG_FC1 | FRAG_LN);
    if (!w->fc2_wf[j]) m &= ~FRAG_FC2;
  }
  // the carried LayerNorm: O on gemm_frag, the statistics buffers, FC1 tiles 64 columns wide, at
  // most 8 frames (the modulate block's 16 rows)
  const int64_t P = (int64_t)w->grid_h * w->grid_w;
  if (!(m & FRAG_O) || !buf->ln_mean || !buf->ln_stats || !buf->ln_mod || Dm % 64 != 0 || (M + P - 1) / P > 8)
    m &= ~FRAG_LN;
  return m;
}

// FC2's split-K count on the fragment-order GEMM: slices of 1024 (4 at d_mlp = 4096)
int frag_fc2_splits(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf) {
  int s = (int)std::max<int64_t>(1, w->d_mlp / 1024);
  return s <= buf->max_splits ? s : -1;
}

// run_sub_block (oasis_inference.py:995-1215) for sub-blocks [j0, j1); sub-block j is
// spatial for even j. The FC2 residual of the last sub-block is left pending. With a
// K/V-cache pass the temporal sub-blocks read and write the cache (run_sub_block_t1,
// oasis_inference.py:1218-1352).
int dit_blocks(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t B, int64_t T, const float* ada,
               int64_t fs, int64_t j0, int64_t j1, Pending* pend, oasis_stream_t stream,
               const KvPass& kv = KvPass()) {
  const int64_t D = w->d_model, H = w->n_heads, Dm = w->d_mlp;
  const int64_t P = (int64_t)w->grid_h * w->grid_w;
  const int64_t M = B * T * P;
  hipStream_t s = (hipStream_t)stream;
  const Plan& pl = plan();
  const int so = pl.splits[ROLE_O] > 0 ? std::min<int>(pl.splits[ROLE_O], buf->max_splits)
                                       : choose_splits(M, D, D, buf->max_splits);
  int sf = pl.splits[ROLE_FC2] > 0 ? std::min<int>(pl.splits[ROLE_FC2], buf->max_splits)
                                   : choose_splits(M, D, Dm, buf->max_splits);
  // fragment order (the FRAG_* bits of the plan): the producer of each chosen operand (residual_ln,
  // the attention kernels, FC1's GELU epilogue) writes it in MFMA fragment order and its projection
  // runs on gemm_frag (O unsplit, FC2 in slices of 1024)
  const int sf_frag = frag_fc2_splits(w, buf);
  const int fg = frag_mask(w, buf, M, j0, j1, sf_frag);
  const bool f_qkv = fg & FRAG_QKV, f_o = fg & FRAG_O, f_fc1 = fg & FRAG_FC1, f_fc2 = fg & FRAG_FC2;
  const bool f_ln = fg & FRAG_LN;
  const int so_use = f_o ? 1 : so;
  if (f_fc2) sf = sf_frag;
  const int64_t FR = buf->frag_rows;

  oasis_epilogue_t qkv = epi_zero();
  qkv.kind = OASIS_EPI_QKV_ROPE;
  qkv.n_heads = (int)H;
  qkv.rows_per_frame = P;
  qkv.frames_per_stream = T;
  const bool fp8 = w->weight_format == OASIS_WEIGHTS_FP8;
  // O and FC2 unsplit with their gated residual in the epilogue where 144 x 128 tiles fill the CUs
  // (unless OASIS_GEMM_PLAN / OASIS_GEMM_PLAN8 place that role themselves)
  const bool unsplit_fill = (M + 143) / 144 * ((D + 127) / 128) >= 256;
  auto unsplit = [&](int role, const int (&tiles)[2]) {
    return unsplit_fill && pl.splits[role] <= 0 && (fp8 ? tiles[1] >= 0 && pl.tile8[role] < 0
                                                           : tiles[0] >= 0 && pl.tile[role] < 0);
  };
  const bool o_res = !f_o && !f_ln && !f_fc1 && unsplit(ROLE_O, pl.o_unsplit);
  const bool fc2_res = !f_fc2 && unsplit(ROLE_FC2, pl.fc2_unsplit);
  oasis_epilogue_t gelu = epi_zero();
  gelu.kind = fp8 ? OASIS_EPI_GELU_TANH_FP8 : (f_fc2 ? OASIS_EPI_GELU_TANH_FRAG : OASIS_EPI_GELU_TANH);
  gelu.out_bf16 = buf->mlp;
  gelu.out_fp8 = buf->mlp8;
  gelu.out_scale = buf->mlp8_scale;
  gelu.ld_scale = Dm / 32;
  gelu.ld_out = Dm;
  const oasis_epilogue_t part = partial_epi(buf->partial, M, D);
  // A operands: bf16 (h, attn, mlp) or, with fp8 weights, fp8 blocks (act8, mlp8)
  uint8_t* a8 = static_cast<uint8_t*>(buf->act8);
  uint8_t* a8s = static_cast<uint8_t*>(buf->act8_scale);
  const void* ln_out = fp8 ? nullptr : buf->h;
  const void* mlp_in = fp8 ? buf->mlp8 : buf->mlp;
  const void* mlp_sc = fp8 ? buf->mlp8_scale : nullptr;

  const bool pf_on = !fp8 && M <= 320;
  const int64_t wbytes[4] = {3 * D * D * 2, D * D * 2, Dm * D * 2, D * Dm * 2};
  for (int64_t j = j0; j < j1; ++j) {
    const bool spatial = (j % 2) == 0;
    const float* a = ada + j * 6 * D;  // shift_a, scale_a+1, gate_a, shift_m, scale_m+1, gate_m
    // the weights the projections below read, for the kernels that read them ahead
    auto weights_of = [&](int64_t i, const void** out) {
      out[0] = f_qkv ? w->qkv_wf[i] : w->qkv_w[i];
      out[1] = (f_o || f_ln) ? w->out_wf[i] : w->out_w[i];
      out[2] = (f_ln || f_fc1) ? w->fc1_wf[i] : w->fc1_w[i];
      out[3] = f_fc2 ? w->fc2_wf[i] : w->fc2_w[i];
    };
    const void* wp[4];
    const void* wn[4] = {nullptr, nullptr, nullptr, nullptr};  // the next sub-block's, if any
    weights_of(j, wp);
    if (j + 1 < w->n_sub) weights_of(j + 1, wn);
    const int pps = M <= 160 ? 0 : 1;
    const int pfl = pl.pf_line[pps];
    const int (&hosts)[4] = pl.pf_host[pps];
    const oasis::Prefetch pf_qkv = prefetch_for(hosts, PF_LN, pf_on, wp, wbytes, pfl, wn);
    const oasis::Prefetch pf_attn = prefetch_for(hosts, PF_ATTN, pf_on, wp, wbytes, pfl, wn);
    const oasis::Prefetch pf_qkvg = prefetch_for(hosts, PF_QKVG, pf_on, wp, wbytes, pfl, wn);
    const oasis::Prefetch pf_og = prefetch_for(hosts, PF_OG, pf_on, wp, wbytes, pfl, wn);
    const oasis::Prefetch pf_fc1g = prefetch_for(hosts, PF_FC1G, pf_on, wp, wbytes, pfl, wn);
    const oasis::Prefetch pf_fc2g = prefetch_for(hosts, PF_FC2G, pf_on, wp, wbytes, pfl, wn);
    // previous FC2 residual (if any) + LN + modulate (oasis_inference.py:1053-1056)
    OASIS_TRY(oasis::residual_ln(buf->x, M, D, buf->partial, pend->n, M * D, pend->bias, pend->gate, fs, P, a + D, a,
                                 fs, (void*)ln_out, fp8 ? a8 : nullptr, a8s, kLnEps, s, f_qkv,
                                 f_ln ? buf->ln_mean : nullptr, &pf_qkv));
    // with OASIS_TEMPORAL_FUSED=1 or 2, two-frame temporal windows (the T = 2 step and the frame's
    // first, cache-filling pass; with 2 also the current-frame passes against the cache): QKV,
    // RoPE and the causal attention in one kernel
    if (!spatial && !fp8 && pl.fused_temporal > 0 && pl.tile[ROLE_QKV] < 0 && P % 16 == 0 &&
        ((kv.mode == KV_NONE && T == 2) || kv.mode == KV_SAVE_T2 || (kv.mode == KV_USE_T1 && pl.fused_temporal > 1))) {
      bf16* kcj = kv.mode == KV_NONE ? nullptr : kv.k + (j / 2) * kv.sub_stride;
      bf16* vcj = kv.mode == KV_NONE ? nullptr : kv.v + (j / 2) * kv.sub_stride;
      OASIS_TRY(oasis::temporal_qkv_attention(static_cast<const bf16*>(buf->h), D,
                                              static_cast<const bf16*>(w->qkv_w[j]), static_cast<bf16*>(buf->attn),
                                              B, kv.mode == KV_USE_T1 ? 1 : 2, P, H, w->t_cos, w->t_sinp, kcj, vcj,
                                              kAttnScale, s));
    } else {
      bf16* kc = nullptr;
      bf16* vc = nullptr;
      int qf = -1;  // temporal query frame (-1: all)
      qkv.q = buf->q;
      qkv.k = buf->k;
      qkv.v = buf->v;
      if (spatial) {  // heads-first per frame: [(b*T + t)*H + h][p][64]
        qkv.s_b = T * H * P * 64;
        qkv.s_t = H * P * 64;
        qkv.s_h = P * 64;
        qkv.s_p = 64;
        qkv.rope_cos = w->s_cos;
        qkv.rope_sinp = w->s_sinp;
        qkv.rope_by_frame = 0;
      } else if (kv.mode == KV_NONE) {  // grouped by position: [b][p][h][t][64]
        qkv.s_b = P * H * T * 64;
        qkv.s_p = H * T * 64;
        qkv.s_h = T * 64;
        qkv.s_t = 64;
        qkv.rope_cos = w->t_cos;
        qkv.rope_sinp = w->t_sinp;
        qkv.rope_by_frame = 1;
      } else {  // the cache's 2-slot layout [b][p][h][2][64]; T=1 passes write one slot
        kc = kv.k + (j / 2) * kv.sub_stride;
        vc = kv.v + (j / 2) * kv.sub_stride;
        const int slot = kv.mode == KV_USE_T1 ? 1 : 0;
        qf = kv.mode == KV_SAVE_T2 ? -1 : slot;
        qkv.s_b = P * H * 2 * 64;
        qkv.s_p = H * 2 * 64;
        qkv.s_h = 2 * 64;
        qkv.s_t = 64;
        qkv.q = static_cast<bf16*>(buf->q) + slot * 64;
        qkv.k = kc + slot * 64;
        qkv.v = vc + slot * 64;
        qkv.rope_cos = w->t_cos + slot * 64;  // RoPE position = slot + t
        qkv.rope_sinp = w->t_sinp + slot * 64;
        qkv.rope_by_frame = 1;
      }
      if (f_qkv)
        OASIS_TRY(oasis::gemm_frag_launch((const bf16*)buf->h, FR, (const bf16*)w->qkv_wf[j], M, 3 * D, D, qkv, 1, s));
      else
        OASIS_TRY(proj(w, ROLE_QKV, j, fp8 ? (const void*)a8 : buf->h, D, a8s, M, 3 * D, D, qkv, pl.tile[ROLE_QKV], 1,
                       s, &pf_qkvg));
      // with fp8 weights the attention writes O's A operand as fp8 blocks itself
      uint8_t* o8 = fp8 ? a8 : nullptr;
      uint8_t* o8s = fp8 ? a8s : nullptr;
      if (spatial)
        OASIS_TRY(oasis::attention(buf->q, buf->k, buf->v, buf->attn, B * T, P, H, kAttnScale, s, f_o, &pf_attn, o8,
                                   o8s));
      else if (kv.mode == KV_NONE)
        OASIS_TRY(oasis::temporal_attention(buf->q, buf->k, buf->v, buf->attn, B, T, P, H, kAttnScale, -1, s, f_o,
                                            &pf_attn, o8, o8s));
      else
        OASIS_TRY(oasis::temporal_attention(buf->q, kc, vc, buf->attn, B, 2, P, H, kAttnScale, qf, s, f_o,
                                            &pf_attn, o8, o8s));
    }
    gelu.bias = w->fc1_b[j];
    if (f_ln) {
      // O + bias + gated residual into x in the epilogue, which also leaves FC1 the centred rows
      // times the modulate scale (fragment order, in h) and their per-32-column sums; FC1 finishes
      // the LayerNorm + modulate (the identity at gemm_frag_kernel)
      oasis_epilogue_t o = epi_zero();
      o.kind = OASIS_EPI_GATED_RES_LN;
      o.bias = w->out_b[j];
      o.out_f32 = buf->x;
      o.out_bf16 = buf->h;
      o.ld_out = D;
      o.gate = a + 2 * D;
      o.gate_fstride = fs;
      o.rows_per_frame = P;
      o.mod_scale = a + 4 * D;
      o.mod_shift = a + 3 * D;
      o.ln_center = buf->ln_mean;
      o.ln_stats = buf->ln_stats;
      o.ln_mod = buf->ln_mod;
      OASIS_TRY(
          oasis::gemm_frag_launch((const bf16*)buf->attn, FR, (const bf16*)w->out_wf[j], M, D, D, o, 1, s, &pf_og));
      oasis_epilogue_t f1 = gelu;
      f1.kind = OASIS_EPI_GELU_TANH_LN;
      f1.rows_per_frame = P;
      f1.ln_stats = buf->ln_stats;
      f1.ln_mod = buf->ln_mod;
      f1.ln_eps = kLnEps;
      f1.out_frag = f_fc2 ? 1 : 0;
      OASIS_TRY(
          oasis::gemm_frag_launch((const bf16*)buf->h, FR, (const bf16*)w->fc1_wf[j], M, Dm, D, f1, 1, s, &pf_fc1g));
    } else if (o_res) {
      // O unsplit with bias + gated residual into x in its epilogue, then LN + modulate alone
      OASIS_TRY(proj(w, ROLE_O, j, fp8 ? (const void*)a8 : buf->attn, D, a8s, M, D, D,
                     gated_res_epi(buf->x, D, w->out_b[j], a + 2 * D, fs, P), pl.o_unsplit[0], 1, s, nullptr,
                     pl.o_unsplit[1]));
      OASIS_TRY(oasis::residual_ln(buf->x, M, D, buf->partial, 0, M * D, nullptr, nullptr, fs, P, a + 4 * D, a + 3 * D,
                                   fs, (void*)ln_out, fp8 ? a8 : nullptr, a8s, kLnEps, s, f_fc1));
      OASIS_TRY(proj(w, ROLE_FC1, j, fp8 ? (const void*)a8 : buf->h, D, a8s, M, Dm, D, gelu, pl.tile[ROLE_FC1], 1, s,
                     &pf_fc1g));
    } else {
      // O projection as split-K partials; bias + gated residual + LN + modulate fused after
      if (f_o)
        OASIS_TRY(oasis::gemm_frag_launch((const bf16*)buf->attn, FR, (const bf16*)w->out_wf[j], M, D, D, part, so_use,
                                          s, &pf_og));
      else
        OASIS_TRY(proj(w, ROLE_O, j, fp8 ? (const void*)a8 : buf->attn, D, a8s, M, D, D, part, pl.tile[ROLE_O], so, s));
      OASIS_TRY(oasis::residual_ln(buf->x, M, D, buf->partial, so_use, M * D, w->out_b[j], a + 2 * D, fs, P, a + 4 * D,
                                   a + 3 * D, fs, (void*)ln_out, fp8 ? a8 : nullptr, a8s, kLnEps, s, f_fc1));
      if (f_fc1)
        OASIS_TRY(oasis::gemm_frag_launch((const bf16*)buf->h, FR, (const bf16*)w->fc1_wf[j], M, Dm, D, gelu, 1, s,
                                          &pf_fc1g));
      else
        OASIS_TRY(proj(w, ROLE_FC1, j, fp8 ? (const void*)a8 : buf->h, D, a8s, M, Dm, D, gelu, pl.tile[ROLE_FC1], 1, s,
                       &pf_fc1g));
    }
    if (fc2_res) {  // FC2 unsplit: its gated residual lands in x, nothing stays pending
      OASIS_TRY(proj(w, ROLE_FC2, j, mlp_in, Dm, mlp_sc, M, D, Dm,
                     gated_res_epi(buf->x, D, w->fc2_b[j], a + 5 * D, fs, P), pl.fc2_unsplit[0], 1, s, nullptr,
                     pl.fc2_unsplit[1]));
      *pend = Pending();
      continue;
    }
    if (f_fc2)
      OASIS_TRY(
          oasis::gemm_frag_launch((const bf16*)buf->mlp, FR, (const bf16*)w->fc2_wf[j], M, D, Dm, part, sf, s, &pf_fc2g));
    else
      OASIS_TRY(proj(w, ROLE_FC2, j, mlp_in, Dm, mlp_sc, M, D, Dm, part, pl.tile[ROLE_FC2], sf, s, &pf_fc2g));
    pend->bias = w->fc2_b[j];
    pend->gate = a + 5 * D;
    pend->n = sf;
  }
  return OASIS_OK;
}

int dit_args(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t B, int64_t T, const float* ada) {
  OASIS_TRY(check_dit(w));
  OASIS_TRY(check_dit_buf(buf, w));
  OASIS_REQUIRE(ada, OASIS_ERR_NULL, "dit: null ada");
  OASIS_REQUIRE(B > 0 && T > 0 && T <= w->t_max, OASIS_ERR_SHAPE, "dit: need B > 0, 0 < T <= t_max (%d)", w->t_max);
  const int64_t M = B * T * (int64_t)w->grid_h * w->grid_w;
  OASIS_REQUIRE(M <= buf->max_rows, OASIS_ERR_SHAPE, "dit: %lld rows exceed the workspace (%lld)", (long long)M,
                (long long)buf->max_rows);
  return OASIS_OK;
}

// final layer (oasis_inference.py:1497-1521): adaLN(2 chunks) + LN + modulate + linear,
// with any pending FC2 residual folded into the LN pass. With chunk set, the DDIM update of
// chunk from the v rows chunk_row0.. (oasis_inference.py:1919-1931) runs in the same launch.
int dit_final(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t M, const float* ada, int64_t fs,
              const Pending& pend, float* v_out, oasis_stream_t stream, float* chunk = nullptr,
              int64_t chunk_row0 = 0, const float* ddim = nullptr) {
  const int64_t D = w->d_model, P = (int64_t)w->grid_h * w->grid_w;
  const float* fa = ada + (int64_t)w->n_sub * 6 * D;  // shift, scale_p1
  return oasis::final_layer(buf->x, M, D, buf->partial, pend.n, M * D, pend.bias, pend.gate, fs, P, fa + D, fa, fs,
                            w->final_w, w->final_b, v_out, kLnEps, (hipStream_t)stream, chunk, chunk_row0, ddim);
}

}  // namespace

namespace {

}  // namespace

extern "C" int oasis_dit_step(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t B, int64_t T,
                              const float* t, const float* action, const float* patches, float* hid, float* cond,
                              float* ada, float* v_out, oasis_stream_t stream) {
  OASIS_TRY(dit_args(w, buf, B, T, ada));
  OASIS_REQUIRE(patches && v_out, OASIS_ERR_NULL, "dit_step: null patches/v_out");
  OASIS_REQUIRE(w->xemb_w && w->xemb_b, OASIS_ERR_NULL, "dit_step: missing patch-embed weights");
  const int64_t R = B * T, D = w->d_model, P = (int64_t)w->grid_h * w->grid_w, NA = ada_width(w);
  OASIS_REQUIRE(R <= 1024, OASIS_ERR_SHAPE, "dit_step: at most 1024 frames per call (got %lld)", (long long)R);
  OASIS_TRY(cond_mlp(w, t, action, R, hid, cond, stream));
  OASIS_TRY(adaln_rows(w, cond, R, ada, (hipStream_t)stream));
  OASIS_TRY(oasis_small_linear(patches, w->patch_dim, B * T * P, w->patch_dim, w->xemb_w, OASIS_F32, 1, D, w->xemb_b,
                               buf->x, D, stream));
  Pending pend;
  OASIS_TRY(dit_blocks(w, buf, B, T, ada, NA, 0, w->n_sub, &pend, stream));
  return dit_final(w, buf, B * T * P, ada, NA, pend, v_out, stream);
}

extern "C" int oasis_dit_sub_blocks(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t B,
                                    int64_t T, const float* ada, int64_t ada_fstride, int64_t j0, int64_t j1,
                                    oasis_stream_t stream) {
  OASIS_TRY(dit_args(w, buf, B, T, ada));
  OASIS_REQUIRE(0 <= j0 && j0 <= j1 && j1 <= w->n_sub, OASIS_ERR_ARG, "dit: sub-block range [%lld, %lld) invalid",
                (long long)j0, (long long)j1);
  Pending pend;
  OASIS_TRY(dit_blocks(w, buf, B, T, ada, ada_fstride, j0, j1, &pend, stream));
  if (pend.n == 0) return OASIS_OK;
  const int64_t M = B * T * (int64_t)w->grid_h * w->grid_w;
  return oasis_residual_ln(buf->x, M, w->d_model, buf->partial, pend.n, M * w->d_model, pend.bias, pend.gate,
                           ada_fstride, (int64_t)w->grid_h * w->grid_w, nullptr, nullptr, 0, nullptr, kLnEps, stream);
}

extern "C" int oasis_dit_final(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t M,
                               const float* ada, int64_t ada_fstride, float* v_out, oasis_stream_t stream) {
  OASIS_TRY(check_dit(w));
  OASIS_TRY(check_dit_buf(buf, w));
  OASIS_REQUIRE(ada && v_out, OASIS_ERR_NULL, "dit_final: null pointer");
  OASIS_REQUIRE(M > 0 && M <= buf->max_rows, OASIS_ERR_SHAPE, "dit_final: bad row count");
  return dit_final(w, buf, M, ada, ada_fstride, Pending(), v_out, stream);
}

extern "C" int oasis_dit_forward(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, int64_t B, int64_t T,
                                 const float* ada, int64_t ada_fstride, float* v_out, oasis_stream_t stream) {
  OASIS_TRY(dit_args(w, buf, B, T, ada));
  OASIS_REQUIRE(v_out, OASIS_ERR_NULL, "dit_forward: null v_out");
  Pending pend;
  OASIS_TRY(dit_blocks(w, buf, B, T, ada, ada_fstride, 0, w->n_sub, &pend, stream));
  return dit_final(w, buf, B * T * (int64_t)w->grid_h * w->grid_w, ada, ada_fstride, pend, v_out, stream);
}

namespace {

int kv_args(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, const oasis_kv_cache_t* kv, int64_t B,
            const float* ada, KvPass* out, int mode) {
  OASIS_TRY(dit_args(w, buf, B, 1, ada));
  OASIS_REQUIRE(kv && kv->k && kv->v, OASIS_ERR_NULL, "kv cache: null pointer");
  OASIS_REQUIRE(B <= kv->max_streams, OASIS_ERR_SHAPE, "kv cache: %lld streams exceed its %lld", (long long)B,
                (long long)kv->max_streams);
  const int64_t P = (int64_t)w->grid_h * w->grid_w;
  OASIS_REQUIRE(w->t_max >= 2, OASIS_ERR_SHAPE, "kv cache: temporal RoPE table needs >= 2 frames");
  OASIS_REQUIRE(2 * B * P <= buf->max_rows, OASIS_ERR_SHAPE,
                "kv cache: the q buffer holds 2 frames per stream; need max_rows >= %lld", (long long)(2 * B * P));
  out->k = static_cast<bf16*>(kv->k);
  out->v = static_cast<bf16*>(kv->v);
  out->sub_stride = kv->max_streams * P * 2 * w->d_model;
  out->mode = mode;
  return OASIS_OK;
}

}  // namespace

extern "C" int oasis_dit_precompute_past(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                                         const oasis_kv_cache_t* kv, int64_t B, const float* ada,
                                         int64_t ada_fstride, oasis_stream_t stream) {
  KvPass kp;
  OASIS_TRY(kv_args(w, buf, kv, B, ada, &kp, KV_SAVE_T1));
  Pending pend;
  return dit_blocks(w, buf, B, 1, ada, ada_fstride, 0, w->n_sub, &pend, stream, kp);
}

extern "C" int oasis_dit_forward_current(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                                         const oasis_kv_cache_t* kv, int64_t B, const float* ada,
                                         int64_t ada_fstride, float* v_out, oasis_stream_t stream) {
  KvPass kp;
  OASIS_TRY(kv_args(w, buf, kv, B, ada, &kp, KV_USE_T1));
  OASIS_REQUIRE(v_out, OASIS_ERR_NULL, "dit_forward_current: null v_out");
  Pending pend;
  OASIS_TRY(dit_blocks(w, buf, B, 1, ada, ada_fstride, 0, w->n_sub, &pend, stream, kp));
  return dit_final(w, buf, B * (int64_t)w->grid_h * w->grid_w, ada, ada_fstride, pend, v_out, stream);
}

namespace {

// vae_decode_forward (oasis_inference.py:1546-1618) + vae_unpatchify for B latents at once: every
// projection runs over B*L tokens, the attention per latent (B frames of L tokens). With pred set,
// the predictor writes its plain rows (acc + bias, unclamped: vae_decode_forward's pred_out) to
// pred[B*L, ld_pred] instead of the unpatchified frames.
int vae_decode(const oasis_vae_weights_t* w, const oasis_vae_buffers_t* buf, int64_t B, const float* latent,
               float* frame, oasis_stream_t stream, float* pred = nullptr, int64_t ld_pred = 0) {
  OASIS_REQUIRE(w && buf && latent && (frame || pred), OASIS_ERR_NULL, "vae_decode: null pointer");
  OASIS_REQUIRE(!pred || ld_pred >= 3LL * w->patch * w->patch, OASIS_ERR_ARG,
                "vae_decode: ld_pred=%lld is below the predictor's %lld columns", (long long)ld_pred,
                3LL * w->patch * w->patch);
  OASIS_REQUIRE(w->depth > 0 && w->depth <= OASIS_MAX_SUB && w->n_heads > 0 && w->d_model == w->n_heads * 64,
                OASIS_ERR_SHAPE, "vae_decode: bad depth/heads/d_model");
  OASIS_REQUIRE(buf->x && buf->h && buf->q && buf->k && buf->v && buf->attn && buf->mlp && buf->partial,
                OASIS_ERR_NULL, "vae_decode: missing buffer");
  OASIS_REQUIRE(buf->max_splits >= 1, OASIS_ERR_ARG, "vae_decode: max_splits must be >= 1");
  OASIS_REQUIRE(w->pq_w && w->pq_b && w->norm_w && w->norm_b && w->pred_w && w->pred_b && w->rope_cos &&
                    w->rope_sinp,
                OASIS_ERR_NULL, "vae_decode: missing weight pointer");
  const int64_t D = w->d_model, H = w->n_heads, Dm = w->d_mlp;
  const int64_t Lf = (int64_t)w->grid_h * w->grid_w;  // tokens per latent
  OASIS_REQUIRE(B > 0 && B * Lf <= buf->max_rows, OASIS_ERR_SHAPE,
                "vae_decode: %lld latents of %lld tokens exceed the workspace (%lld rows)", (long long)B,
                (long long)Lf, (long long)buf->max_rows);
  const int64_t L = B * Lf;  // rows of every projection
  hipStream_t s = (hipStream_t)stream;
  const Plan& pl = plan();
  const int sp = pl.splits[ROLE_VO] > 0 ? std::min<int>(pl.splits[ROLE_VO], buf->max_splits)
                                        : choose_splits(L, D, D, buf->max_splits);
  const int sf = pl.splits[ROLE_VFC2] > 0 ? std::min<int>(pl.splits[ROLE_VFC2], buf->max_splits)
                                          : choose_splits(L, D, Dm, buf->max_splits);
  OASIS_TRY(oasis_small_linear(latent, w->latent_dim, L, w->latent_dim, w->pq_w, OASIS_BF16, 0, D, w->pq_b, buf->x, D,
                               stream));

  oasis_epilogue_t qkv = epi_zero();
  qkv.kind = OASIS_EPI_QKV_ROPE;
  qkv.n_heads = (int)H;
  qkv.q = buf->q;
  qkv.k = buf->k;
  qkv.v = buf->v;
  qkv.rows_per_frame = Lf;  // latent b = row / Lf, heads-first per latent: [(b*H + h)][Lf][64]
  qkv.frames_per_stream = 1;
  qkv.s_b = H * Lf * 64;
  qkv.s_t = 0;
  qkv.s_h = Lf * 64;
  qkv.s_p = 64;
  qkv.rope_cos = w->rope_cos;
  qkv.rope_sinp = w->rope_sinp;
  oasis_epilogue_t gelu = epi_zero();
  gelu.kind = OASIS_EPI_GELU_ERF;
  gelu.out_bf16 = buf->mlp;
  gelu.ld_out = Dm;
  const oasis_epilogue_t part = partial_epi(buf->partial, L, D);
  // batched decodes whose unsplit 144 x 128 tiles fill the CUs: O and FC2 unsplit (as dit_blocks)
  const bool unsplit_fill = (L + 143) / 144 * ((D + 127) / 128) >= 256;
  const bool o_res = unsplit_fill && pl.tile[ROLE_VO] < 0 && pl.splits[ROLE_VO] <= 0 && pl.o_unsplit[0] >= 0;
  const bool fc2_res = unsplit_fill && pl.tile[ROLE_VFC2] < 0 && pl.splits[ROLE_VFC2] <= 0 && pl.fc2_unsplit[0] >= 0;

  Pending pend;
  const int64_t wbytes[4] = {3 * D * D * 2, D * D * 2, Dm * D * 2, D * Dm * 2};
  for (int i = 0; i < w->depth; ++i) {
    OASIS_REQUIRE(w->n1_w[i] && w->n1_b[i] && w->qkv_w[i] && w->qkv_b[i] && w->proj_w[i] && w->proj_b[i] &&
                      w->n2_w[i] && w->n2_b[i] && w->fc1_w[i] && w->fc1_b[i] && w->fc2_w[i] && w->fc2_b[i],
                  OASIS_ERR_NULL, "vae_decode: missing weights of block %d", i);
    // weights read ahead, as in dit_blocks
    const void* const wp[4] = {w->qkv_w[i], w->proj_w[i], w->fc1_w[i], w->fc2_w[i]};
    const oasis::Prefetch pf_qkv = prefetch_for(kVaePrefetch, PF_LN, L < 2048, wp, wbytes, pl.pf_line[2]);
    const oasis::Prefetch pf_attn = prefetch_for(kVaePrefetch, PF_ATTN, L < 2048, wp, wbytes, pl.pf_line[2]);
    // x + attn(LN(x)); x + MLP(LN(x)) (oasis_inference.py:1557-1608)
    OASIS_TRY(oasis::residual_ln(buf->x, L, D, buf->partial, pend.n, L * D, pend.bias, nullptr, 0, L, w->n1_w[i],
                                 w->n1_b[i], 0, buf->h, nullptr, nullptr, kLnEps, s, false, nullptr, &pf_qkv));
    qkv.bias = w->qkv_b[i];
    OASIS_TRY(oasis::gemm_launch_cfg((const bf16*)buf->h, D, (const bf16*)w->qkv_w[i], D, L, 3 * D, D, qkv,
                                     pl.tile[ROLE_VQKV], 1, s));
    OASIS_TRY(oasis::attention(buf->q, buf->k, buf->v, buf->attn, B, Lf, H, kAttnScale, s, false, &pf_attn));
    if (o_res) {  // unsplit, the residual added in the epilogue (as the DiT's large-token passes)
      OASIS_TRY(oasis::gemm_launch_cfg((const bf16*)buf->attn, D, (const bf16*)w->proj_w[i], D, L, D, D,
                                       residual_epi(buf->x, D, w->proj_b[i]), pl.o_unsplit[0], 1, s));
      OASIS_TRY(oasis_residual_ln(buf->x, L, D, nullptr, 0, L * D, nullptr, nullptr, 0, L, w->n2_w[i], w->n2_b[i], 0,
                                  buf->h, kLnEps, stream));
    } else {
      OASIS_TRY(oasis::gemm_launch_cfg((const bf16*)buf->attn, D, (const bf16*)w->proj_w[i], D, L, D, D, part,
                                       pl.tile[ROLE_VO], sp, s));
      OASIS_TRY(oasis_residual_ln(buf->x, L, D, buf->partial, sp, L * D, w->proj_b[i], nullptr, 0, L, w->n2_w[i],
                                  w->n2_b[i], 0, buf->h, kLnEps, stream));
    }
    gelu.bias = w->fc1_b[i];
    OASIS_TRY(oasis::gemm_launch_cfg((const bf16*)buf->h, D, (const bf16*)w->fc1_w[i], D, L, Dm, D, gelu,
                                     pl.tile[ROLE_VFC1], 1, s));
    if (fc2_res) {
      OASIS_TRY(oasis::gemm_launch_cfg((const bf16*)buf->mlp, Dm, (const bf16*)w->fc2_w[i], Dm, L, D, Dm,
                                       residual_epi(buf->x, D, w->fc2_b[i]), pl.fc2_unsplit[0], 1, s));
      pend = Pending();
    } else {
      OASIS_TRY(oasis::gemm_launch_cfg((const bf16*)buf->mlp, Dm, (const bf16*)w->fc2_w[i], Dm, L, D, Dm, part,
                                       pl.tile[ROLE_VFC2], sf, s));
      pend.bias = w->fc2_b[i];
      pend.n = sf;
    }
  }
  OASIS_TRY(oasis_residual_ln(buf->x, L, D, buf->partial, pend.n, L * D, pend.bias, nullptr, 0, L, w->norm_w, w->norm_b,
                              0, buf->h, kLnEps, stream));
  oasis_epilogue_t pe = epi_zero();
  pe.bias = w->pred_b;
  if (pred) {
    pe.kind = OASIS_EPI_STORE_F32;
    pe.out_f32 = pred;
    pe.ld_out = ld_pred;
  } else {
    pe.kind = OASIS_EPI_UNPATCHIFY;
    pe.out_f32 = frame;
    pe.rows_per_frame = Lf;
    pe.unpatch_grid_w = w->grid_w;
    pe.unpatch_patch = w->patch;
    pe.unpatch_channels = 3;
  }
  return oasis::gemm_launch((const bf16*)buf->h, D, (const bf16*)w->pred_w, D, L, 3LL * w->patch * w->patch, D, pe,
                            s);
}

}  // namespace

extern "C" int oasis_vae_decode(const oasis_vae_weights_t* w, const oasis_vae_buffers_t* buf, const float* latent,
                                float* frame, oasis_stream_t stream) {
  OASIS_REQUIRE(frame, OASIS_ERR_NULL, "vae_decode: null frame");
  return vae_decode(w, buf, 1, latent, frame, stream);
}

extern "C" int oasis_vae_decode_batch(const oasis_vae_weights_t* w, const oasis_vae_buffers_t* buf, int64_t B,
                                      const float* latents, float* frames, oasis_stream_t stream) {
  OASIS_REQUIRE(frames, OASIS_ERR_NULL, "vae_decode_batch: null frames");
  return vae_decode(w, buf, B, latents, frames, stream);
}

extern "C" int oasis_vae_decode_patches(const oasis_vae_weights_t* w, const oasis_vae_buffers_t* buf, int64_t B,
                                        const float* latents, float* pred_out, int64_t ld_pred,
                                        oasis_stream_t stream) {
  OASIS_REQUIRE(pred_out, OASIS_ERR_NULL, "vae_decode_patches: null pred_out");
  return vae_decode(w, buf, B, latents, nullptr, stream, pred_out, ld_pred);
}

namespace {

// the bridge of chunks[0, n) into latents, then their decodes, as batches of as many latents as the
// VAE workspace holds (latent: [that many, 4P, latent_dim] scratch)
int decode_chunks(const oasis_dit_weights_t* w, const oasis_vae_weights_t* vw, const oasis_vae_buffers_t* vbuf,
                  int64_t n, const float* chunks, float* latent, float* frames, oasis_stream_t stream) {
  const int64_t P = (int64_t)w->grid_h * w->grid_w, C = w->patch_dim / 4, fsz = (int64_t)w->patch_dim * P;
  const int64_t Lf = (int64_t)vw->grid_h * vw->grid_w, lsz = Lf * vw->latent_dim;
  const int64_t frame_elems = 3LL * vw->grid_h * vw->patch * vw->grid_w * vw->patch;
  const int64_t per = std::max<int64_t>(1, vbuf->max_rows / Lf);
  for (int64_t f0 = 0; f0 < n; f0 += per) {
    const int64_t b = std::min(per, n - f0);
    for (int64_t i = 0; i < b; ++i)
      OASIS_TRY(oasis_bridge(chunks + (f0 + i) * fsz, latent + i * lsz, w->grid_h, w->grid_w, C, vw->latent_dim,
                             kInvScaling, stream));
    OASIS_TRY(vae_decode(vw, vbuf, b, latent, frames + f0 * frame_elems, stream));
  }
  return OASIS_OK;
}

}  // namespace

namespace {

// The n_steps DDIM steps of one generated frame whose context is already embedded in
// ctx_z; ada holds the frame's conditioning rows (0 context, 1 + i step i). With a K/V
// cache, step 0 runs at T=2 storing the context's temporal K/V and later steps run the
// generated frame alone at T=1. chunk is updated in place.
int frame_steps(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, const oasis_kv_cache_t* kv,
                float* chunk, const float* ctx_z, const float* ada, int64_t n_steps, const float* coeffs,
                float* v_out, oasis_stream_t stream) {
  const int64_t D = w->d_model, P = (int64_t)w->grid_h * w->grid_w, NA = ada_width(w);
  hipStream_t s = (hipStream_t)stream;
  KvPass save, use;
  if (kv) {
    OASIS_TRY(kv_args(w, buf, kv, 1, ada, &save, KV_SAVE_T2));
    use = save;
    use.mode = KV_USE_T1;
  }
  for (int64_t i = 0; i < n_steps; ++i) {
    const bool t1 = kv && i > 0;  // K/V cache filled by step 0: the current frame alone
    const float* c = coeffs + 6 * i;
    Pending pend;
    if (t1) {
      OASIS_TRY(oasis_small_linear(chunk, w->patch_dim, P, w->patch_dim, w->xemb_w, OASIS_F32, 1, D, w->xemb_b, buf->x, D,
                                   stream));
      const float* ada_cur = ada + (1 + i) * NA;  // the generated frame's rows at step i
      OASIS_TRY(dit_blocks(w, buf, 1, 1, ada_cur, NA, 0, w->n_sub, &pend, stream, use));
      OASIS_TRY(dit_final(w, buf, P, ada_cur, NA, pend, v_out, stream, chunk, 0, c));
      continue;
    }
    // z = [context frame; patch-embedded chunk] (oasis_inference.py:1911-1913)
    if (hipMemcpyAsync(buf->x, ctx_z, P * D * sizeof(float), hipMemcpyDeviceToDevice, s) != hipSuccess)
      return oasis::check_launch("ddim_frame context copy");
    OASIS_TRY(oasis_small_linear(chunk, w->patch_dim, P, w->patch_dim, w->xemb_w, OASIS_F32, 1, D, w->xemb_b,
                                 buf->x + P * D, D, stream));
    const int64_t fs = (1 + i) * NA;  // frame 0 -> ada row 0, frame 1 -> ada row 1 + i
    OASIS_TRY(dit_blocks(w, buf, 1, 2, ada, fs, 0, w->n_sub, &pend, stream, kv ? save : KvPass()));
    OASIS_TRY(dit_final(w, buf, 2 * P, ada, fs, pend, v_out, stream, chunk, P, c));
  }
  return OASIS_OK;
}

int frame_args(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf, const oasis_vae_weights_t* vw,
               int64_t n_steps) {
  OASIS_TRY(check_dit(w));
  OASIS_TRY(check_dit_buf(buf, w));
  OASIS_REQUIRE(vw, OASIS_ERR_NULL, "ddim_frame: null VAE weights");
  OASIS_REQUIRE(n_steps > 0 && n_steps <= 15, OASIS_ERR_ARG, "ddim_frame: n_steps must be in [1, 15]");
  OASIS_REQUIRE(w->xemb_w && w->xemb_b, OASIS_ERR_NULL, "ddim_frame: missing patch-embed weights");
  OASIS_REQUIRE(w->t_max >= 2, OASIS_ERR_SHAPE, "ddim_frame: temporal RoPE table needs >= 2 frames");
  const int64_t P = (int64_t)w->grid_h * w->grid_w, C = w->patch_dim / 4;
  OASIS_REQUIRE(2 * P <= buf->max_rows, OASIS_ERR_SHAPE, "ddim_frame: workspace too small for T=2");
  OASIS_REQUIRE((int64_t)vw->grid_h * vw->grid_w == 4 * P && vw->latent_dim >= C, OASIS_ERR_SHAPE,
                "ddim_frame: VAE grid must be the 2x-upsampled DiT grid");
  return OASIS_OK;
}

}  // namespace

extern "C" int oasis_ddim_frame(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                                const oasis_vae_weights_t* vw, const oasis_vae_buffers_t* vbuf,
                                const oasis_kv_cache_t* kv, float* chunk, const float* ctx_patches, const float* t,
                                const float* action, int64_t n_steps, const float* coeffs, float* hid, float* cond,
                                float* ada, float* ctx_z, float* v_out, float* latent, float* frame,
                                oasis_stream_t stream) {
  OASIS_TRY(frame_args(w, buf, vw, n_steps));
  OASIS_REQUIRE(vbuf && chunk && ctx_patches && coeffs && ada && ctx_z && v_out && latent && frame,
                OASIS_ERR_NULL, "ddim_frame: null pointer");
  const int64_t D = w->d_model, P = (int64_t)w->grid_h * w->grid_w, C = w->patch_dim / 4;
  // conditioning rows: 0 = context frame, 1 + i = generated frame at step i; one adaLN pass
  // covers all rows
  OASIS_TRY(cond_mlp(w, t, action, 1 + n_steps, hid, cond, stream));
  OASIS_TRY(adaln_rows(w, cond, 1 + n_steps, ada, (hipStream_t)stream));
  OASIS_TRY(oasis_small_linear(ctx_patches, w->patch_dim, P, w->patch_dim, w->xemb_w, OASIS_F32, 1, D, w->xemb_b, ctx_z,
                               D, stream));
  OASIS_TRY(frame_steps(w, buf, kv, chunk, ctx_z, ada, n_steps, coeffs, v_out, stream));
  OASIS_TRY(oasis_bridge(chunk, latent, w->grid_h, w->grid_w, C, vw->latent_dim, kInvScaling, stream));
  return oasis_vae_decode(vw, vbuf, latent, frame, stream);
}

extern "C" int oasis_video_frames(const oasis_dit_weights_t* w, const oasis_dit_buffers_t* buf,
                                  const oasis_vae_weights_t* vw, const oasis_vae_buffers_t* vbuf,
                                  const oasis_kv_cache_t* kv, int64_t n_frames, float* chunks,
                                  const float* ctx_patches, const float* t, const float* action, int64_t n_steps,
                                  const float* coeffs, float* hid, float* cond, float* ada, float* ctx_z,
                                  float* v_out, float* latent, float* frames, oasis_stream_t stream) {
  OASIS_TRY(frame_args(w, buf, vw, n_steps));
  const bool decode = frames != nullptr;  // frames == NULL: the DiT half only
  OASIS_REQUIRE(chunks && ctx_patches && t && action && coeffs && hid && cond && ada && ctx_z && v_out &&
                    (!decode || (vbuf && latent)),
                OASIS_ERR_NULL, "video_frames: null pointer");
  OASIS_REQUIRE(n_frames > 0 && n_frames <= OASIS_MAX_SUB, OASIS_ERR_ARG, "video_frames: n_frames must be in [1, %d]",
                OASIS_MAX_SUB);
  const int64_t D = w->d_model, P = (int64_t)w->grid_h * w->grid_w, NA = ada_width(w);
  const int64_t R = 1 + n_steps, fsz = (int64_t)w->patch_dim * P;
  hipStream_t s = (hipStream_t)stream;
  // every frame's conditioning rows at once: frame f's rows at f*R (context, then step i)
  OASIS_TRY(cond_mlp(w, t, action, n_frames * R, hid, cond, stream));
  OASIS_TRY(adaln_rows(w, cond, n_frames * R, ada, s));
  for (int64_t f = 0; f < n_frames; ++f) {
    // context = the previous frame's denoised latent (the rolled context window)
    const float* ctx = f == 0 ? ctx_patches : chunks + (f - 1) * fsz;
    OASIS_TRY(oasis_small_linear(ctx, w->patch_dim, P, w->patch_dim, w->xemb_w, OASIS_F32, 1, D, w->xemb_b, ctx_z, D,
                                 stream));
    OASIS_TRY(frame_steps(w, buf, kv, chunks + f * fsz, ctx_z, ada + f * R * NA, n_steps, coeffs, v_out,
                          stream));
  }
  // the bridges + decodes after the last frame, batched
  if (decode) OASIS_TRY(decode_chunks(w, vw, vbuf, n_frames, chunks, latent, frames, stream));
  return OASIS_OK;
}

extern "C" int oasis_video_decode(const oasis_dit_weights_t* w, const oasis_vae_weights_t* vw,
                                  const oasis_vae_buffers_t* vbuf, int64_t n_frames, const float* chunks, float* latent,
                                  float* frames, oasis_stream_t stream) {
  OASIS_TRY(check_dit(w));
  OASIS_REQUIRE(vw && vbuf && chunks && latent && frames, OASIS_ERR_NULL, "video_decode: null pointer");
  OASIS_REQUIRE(n_frames > 0 && n_frames <= OASIS_MAX_SUB, OASIS_ERR_ARG, "video_decode: n_frames must be in [1, %d]",
                OASIS_MAX_SUB);
  const int64_t P = (int64_t)w->grid_h * w->grid_w, C = w->patch_dim / 4;
  OASIS_REQUIRE((int64_t)vw->grid_h * vw->grid_w == 4 * P && vw->latent_dim >= C, OASIS_ERR_SHAPE,
                "video_decode: VAE grid must be the 2x-upsampled DiT grid");
  return decode_chunks(w, vw, vbuf, n_frames, chunks, latent, frames, stream);
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
