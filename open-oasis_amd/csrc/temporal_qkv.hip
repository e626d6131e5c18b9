// Temporal sub-block front half for two-frame windows, in one kernel: the QKV projection,
// the temporal RoPE and the causal attention over the two frames of each (stream, position,
// head). It replaces the QKV GEMM + temporal attention pair of the temporal sub-block
// (run_sub_block: qkv linear, rope_temporal and sdpa_causal, oasis_inference.py:1060-1151;
// the K/V-cache variant run_sub_block_t1, oasis_inference.py:1218-1352) when the window is
// two frames, the case of the DiT step (T = 2) and of the K/V-cache steps (T = 1 against the
// cached context frame).
//
// A workgroup (8 or 12 waves) owns 16 positions of one stream and one head:
//   - A tile: the LN output rows of those 16 positions, in both frames (T = 2, 32 rows) or in
//     the current frame (T = 1, 16 rows);
//   - B tile: the head's 64 q, 64 k and 64 v weight rows (192 rows gathered from the
//     [3D, D] QKV weight);
//   - direct-to-LDS K pipeline with the same swizzled 128-byte rows as the projection GEMMs.
// The epilogue stages the fp32 tile in LDS; 16 lanes per position, 4 head dims per lane:
// RoPE on q and k (position = frame index), q / k / v rounded to bf16 as the unfused path
// stores them, then query frame 0 sees only key 0 (output = v0) and query frame 1 takes the
// softmax over keys 0 and 1, with the 64-dim dot products reduced over the 16 lanes.
// With a K/V cache ([b][p][h][2][64]): T = 2 also stores both frames' rotated K and V in slots
// 0 and 1; T = 1 reads slot 0 (the context frame) and rotates the current frame as position 1.
#include "oasis_common.h"
#include "gemm_epilogue.h"

namespace {

constexpr float kLog2e = 1.4426950408889634f;

struct TqkvArgs {
  const bf16* A;  // LN output [rows, lda]
  int64_t lda;
  const bf16* W;  // QKV weight [3D, D]
  bf16* out;      // attention output [rows, D], token-major
  const float* cos;   // temporal RoPE tables [t][64]
  const float* sinp;
  bf16* kc;  // K/V cache (nullptr: none)
  bf16* vc;
  int P, H, D, T, G;  // positions per frame, heads, model width, frames in the window, P / 16
  float scale_log2;
};

__device__ __forceinline__ void rope4(float* x, const float* c, const float* s) {
  float r[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) r[j] = x[j] * c[j] + x[j ^ 1] * s[j];
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = bf2f(f2bf(r[j]));
}

__device__ __forceinline__ void load4f(const float* p, float* v) {
  const f32x4 t = *reinterpret_cast<const f32x4*>(p);
  v[0] = t[0];
  v[1] = t[1];
  v[2] = t[2];
  v[3] = t[3];
}

__device__ __forceinline__ void round4(float* v) {
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = bf2f(f2bf(v[j]));
}

__device__ __forceinline__ void store4bf(bf16* p, const float* v) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{f2bf(v[0]), f2bf(v[1]), f2bf(v[2]), f2bf(v[3])};
}

__device__ __forceinline__ void load4bf(const bf16* p, float* v) {
  const bf16x4 t = *reinterpret_cast<const bf16x4*>(p);
#pragma unroll
  for (int j = 0; j < 4; ++j) v[j] = bf2f(t[j]);
}

// BM = 16 * T rows (positions x frames), BN = 192 gathered weight rows, WM x WN waves.
template <int BM, int WM, int WN, int STAGES>
__global__ __launch_bounds__(WM * WN * 64) void tqkv_kernel(TqkvArgs a) {
  constexpr int NW = WM * WN, BN = 192, TM = BM / WM, TN = BN / WN, FM = TM / 16, FN = TN / 16;
  static_assert(FM * 16 == TM && FN * 16 == TN, "wave tiles of whole 16 x 16 blocks");
  constexpr int ROWB = 128;                       // bytes per LDS row: 64 bf16 of K
  constexpr int NBLK = (BM + BN) / 8;             // 1 KB blocks (8 rows) per stage
  constexpr int LPW = (NBLK + NW - 1) / NW;
  constexpr int STAGE_BYTES = (BM + BN) * ROWB;
  constexpr int RING = STAGES * STAGE_BYTES;
  constexpr int CP = BN + 4;                      // fp32 pitch of the staged tile
  constexpr int C_BYTES = BM * CP * 4;
  constexpr int SMEM = RING > C_BYTES ? RING : C_BYTES;
  static_assert(SMEM <= 160 * 1024, "LDS");
  static_assert((STAGES - 2) * LPW <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  // the wave index read back as a scalar, so that the load bases built from it stay in SGPRs
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;
  // position groups run fastest, so one XCD's consecutive workgroups share a few heads' weights
  const int id = xcd_remap(blockIdx.x, gridDim.x);
  const int pg = id % a.G, rest = id / a.G;
  const int h = rest % a.H, b = rest / a.H;
  const int64_t m_base = ((int64_t)b * a.T) * a.P + pg * 16;  // row of (frame f, position i): m_base + f P + i

  // buffer loads: scalar bases (the group's first A row, head h's first q weight row), the K tile
  // as a scalar offset, 32-bit lane offsets (T frames of P rows of A; the q, k, v row blocks of W)
  const __amdgpu_buffer_rsrc_t Ars = buffer_rsrc(a.A + m_base * a.lda);
  const __amdgpu_buffer_rsrc_t Wrs = buffer_rsrc(a.W + (int64_t)h * 64 * a.D);
  uint32_t off[LPW];
  int dst[LPW];
  bool from_a[LPW];
#pragma unroll
  for (int u = 0; u < LPW; ++u) {
    const int blk = min(wave * LPW + u, NBLK - 1);
    const int r = blk * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    from_a[u] = blk * 8 < BM;  // wave-uniform: BM is a multiple of 16
    if (from_a[u]) {
      off[u] = (uint32_t)((((int64_t)(r >> 4) * a.P + (r & 15)) * a.lda + c * 8) * 2);
    } else {
      const int cc = r - BM;  // q, k, v rows of head h
      off[u] = (uint32_t)((((int64_t)(cc >> 6) * a.D + (cc & 63)) * a.D + c * 8) * 2);
    }
    dst[u] = blk * 1024;
  }
  auto issue = [&](int kt, int buf) {
    char* base = smem + buf * STAGE_BYTES;
#pragma unroll
    for (int u = 0; u < LPW; ++u) buffer_load_lds16(from_a[u] ? Ars : Wrs, off[u], kt * 128, base + dst[u]);
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, g = lane >> 4;
  auto compute = [&](int buf) {
    const char* base = smem + buf * STAGE_BYTES;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 4 + g;
      bf16x8 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = wm * TM + i * 16 + lr;
        af[i] = *reinterpret_cast<const bf16x8*>(base + r * ROWB + ((c ^ ((r >> 1) & 7)) << 4));
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int r = BM + wn * TN + j * 16 + lr;
        bfr[j] = *reinterpret_cast<const bf16x8*>(base + r * ROWB + ((c ^ ((r >> 1) & 7)) << 4));
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(af[i], bfr[j], acc[i][j]);
    }
  };

  // vmcnt <= (STAGES - 2) * LPW: every load of the oldest in-flight stage has landed
  constexpr int VM = (STAGES - 2) * LPW;
  constexpr int WAIT = (VM & 15) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8);
  const int nk = a.D / 64;
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue(min(s, nk - 1), s);
  for (int k = 0; k < nk; ++k) {
    __builtin_amdgcn_s_waitcnt(WAIT);
    __builtin_amdgcn_s_barrier();
    issue(min(k + STAGES - 1, nk - 1), (k + STAGES - 1) % STAGES);  // into the buffer read at k - 1
    compute(k % STAGES);
  }
  __builtin_amdgcn_s_waitcnt(0);  // the clamped tail loads must land before the ring is reused
  __syncthreads();

  float* Cs = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) Cs[(wm * TM + i * 16 + g * 4 + r) * CP + wn * TN + j * 16 + lr] = acc[i][j][r];
  __syncthreads();
  if (tid >= 256) return;  // whole waves: the 16-lane groups below stay intact

  // 16 lanes per position (i), 4 head dims per lane (d)
  const int i = tid >> 4, d = (tid & 15) * 4;
  const int p = pg * 16 + i;
  const float* row1 = Cs + (BM - 16 + i) * CP;  // the current (last) frame
  float q1[4], k1[4], v1[4], k0[4], v0[4];
  load4f(row1 + d, q1);
  load4f(row1 + 64 + d, k1);
  load4f(row1 + 128 + d, v1);
  {  // the current frame is RoPE position 1 in both windows
    float c[4], s[4];
    load4f(a.cos + 64 + d, c);
    load4f(a.sinp + 64 + d, s);
    rope4(q1, c, s);
    rope4(k1, c, s);
  }
  round4(v1);
  const int64_t cbase = (((int64_t)b * a.P + p) * a.H + h) * 128 + d;  // cache slot 0 of (b, p, h)
  if (BM == 32) {
    const float* row0 = Cs + i * CP;
    load4f(row0 + 64 + d, k0);
    load4f(row0 + 128 + d, v0);
    float c[4], s[4];
    load4f(a.cos + d, c);
    load4f(a.sinp + d, s);
    rope4(k0, c, s);
    round4(v0);
    if (a.kc) {
      store4bf(a.kc + cbase, k0);
      store4bf(a.vc + cbase, v0);
      store4bf(a.kc + cbase + 64, k1);
      store4bf(a.vc + cbase + 64, v1);
    }
  } else {
    load4bf(a.kc + cbase, k0);
    load4bf(a.vc + cbase, v0);
  }
  float d10 = 0.f, d11 = 0.f;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    d10 += q1[j] * k0[j];
    d11 += q1[j] * k1[j];
  }
  d10 = row16_sum(d10);
  d11 = row16_sum(d11);
  const float x0 = d10 * a.scale_log2, x1 = d11 * a.scale_log2;
  const float mx = fmaxf(x0, x1);
  const float p0 = exp2f(x0 - mx), p1 = exp2f(x1 - mx);
  const float inv = 1.0f / (p0 + p1);
  float o1[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) o1[j] = (p0 * v0[j] + p1 * v1[j]) * inv;
  const int64_t col = (int64_t)h * 64 + d;
  if (BM == 32) store4bf(a.out + (m_base + i) * a.D + col, v0);  // query frame 0: its one key
  store4bf(a.out + (m_base + (int64_t)(BM / 16 - 1) * a.P + i) * a.D + col, o1);
}

}  // namespace

namespace oasis {

int temporal_qkv_attention(const bf16* A, int64_t lda, const bf16* W, bf16* out, int64_t B, int64_t T, int64_t P,
                           int64_t H, const float* t_cos, const float* t_sinp, bf16* kc, bf16* vc, float scale,
                           hipStream_t stream) {
  OASIS_REQUIRE(A && W && out && t_cos && t_sinp, OASIS_ERR_NULL, "temporal_qkv: null pointer");
  OASIS_REQUIRE(T == 2 || (T == 1 && kc && vc), OASIS_ERR_ARG,
                "temporal_qkv: T must be 2, or 1 with the K/V cache of the context frame");
  OASIS_REQUIRE((kc == nullptr) == (vc == nullptr), OASIS_ERR_ARG, "temporal_qkv: K and V cache go together");
  OASIS_REQUIRE(oasis_aligned(16, A, W, out, t_cos, t_sinp) && oasis_aligned(8, kc, vc), OASIS_ERR_ARG,
                "temporal_qkv: misaligned pointer");
  OASIS_REQUIRE(B > 0 && P > 0 && P % 16 == 0 && H > 0 && H * 64 <= 4096 && lda >= H * 64 && lda % 8 == 0,
                OASIS_ERR_SHAPE, "temporal_qkv: need P %% 16 == 0, D = 64 H <= 4096, lda >= D");
  OASIS_REQUIRE(B * T * P * lda < (1ll << 31) && B * (P / 16) * H < (1ll << 31), OASIS_ERR_SHAPE,
                "temporal_qkv: shape too large");
  TqkvArgs a;
  a.A = A;
  a.lda = lda;
  a.W = W;
  a.out = out;
  a.cos = t_cos;
  a.sinp = t_sinp;
  a.kc = kc;
  a.vc = vc;
  a.P = (int)P;
  a.H = (int)H;
  a.D = (int)(H * 64);
  a.T = (int)T;
  a.G = (int)(P / 16);
  a.scale_log2 = scale * kLog2e;
  const dim3 grid((unsigned)(B * (P / 16) * H));
  // 8 waves for the two-frame tile (2 x 4: 16 rows x 48 columns each), 12 for the one-frame
  // tile (16 rows x 16 columns each): 2-3 waves per SIMD hide the K pipeline's latency
  if (T == 2)
    hipLaunchKernelGGL((tqkv_kernel<32, 2, 4, 4>), grid, dim3(512), 0, stream, a);
  else
    hipLaunchKernelGGL((tqkv_kernel<16, 1, 12, 3>), grid, dim3(768), 0, stream, a);
  return check_launch("temporal_qkv");
}

}  // namespace oasis

extern "C" int oasis_temporal_qkv_attention(const void* h, int64_t ldh, const void* w_qkv, void* out, int64_t B,
                                            int64_t T, int64_t P, int64_t n_heads, const float* t_cos,
                                            const float* t_sinp, void* k_cache, void* v_cache, float scale,
                                            oasis_stream_t stream) {
  return oasis::temporal_qkv_attention(static_cast<const bf16*>(h), ldh, static_cast<const bf16*>(w_qkv),
                                       static_cast<bf16*>(out), B, T, P, n_heads, t_cos, t_sinp,
                                       static_cast<bf16*>(k_cache), static_cast<bf16*>(v_cache), scale,
                                       static_cast<hipStream_t>(stream));
}
