// Elementwise and small utility kernels: the reference's elementwise surface
// (silu, adaln_modulate, gated_residual), the DDIM update, the DiT->VAE bridge,
// VAE unpatchify, the timestep embedding, small-K fp32 projections, the reference
// adaln_matmul_expand and the standalone RoPE + head-split kernel.
//
// All of these are HBM-bound; they use grid-stride loops with one element (or one
// 16-byte vector of each operand) per thread step and coalesced accesses.
#include <algorithm>

#include "oasis_common.h"

namespace {

template <typename T>
__device__ __forceinline__ float ld(const T* p, int64_t i);
template <>
__device__ __forceinline__ float ld<float>(const float* p, int64_t i) { return p[i]; }
template <>
__device__ __forceinline__ float ld<bf16>(const bf16* p, int64_t i) { return bf2f(p[i]); }

template <typename T>
__device__ __forceinline__ void st(T* p, int64_t i, float v);
template <>
__device__ __forceinline__ void st<float>(float* p, int64_t i, float v) { p[i] = v; }
template <>
__device__ __forceinline__ void st<bf16>(bf16* p, int64_t i, float v) { p[i] = f2bf(v); }

enum { EW_SILU = 0, EW_MODULATE = 1, EW_GATED = 2, EW_BIAS_GATED = 3 };

template <int OP>
__device__ __forceinline__ float ew_op(float a, float b, float c, float d) {
  if (OP == EW_SILU) return silu(a);
  if (OP == EW_MODULATE) return a * (c + 1.0f) + b;  // x * (scale + 1) + shift ; a=x b=shift c=scale
  if (OP == EW_GATED) return a + b * c;              // residual + x * gate ; a=res b=x c=gate
  return a + (b + c) * d;                            // residual + (x + bias) * gate ; a=res b=x c=bias d=gate
}

// one element per thread step (any alignment)
template <typename T, int OP>
__global__ void ew_kernel(const T* a, const T* b, const T* c, const T* d, T* out, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const float vb = OP != EW_SILU ? ld<T>(b, i) : 0.f, vc = OP != EW_SILU ? ld<T>(c, i) : 0.f;
    const float vd = OP == EW_BIAS_GATED ? ld<T>(d, i) : 0.f;
    st<T>(out, i, ew_op<OP>(ld<T>(a, i), vb, vc, vd));
  }
}

template <typename T>
struct Vec16;
template <>
struct Vec16<float> {
  using V = f32x4;
  static constexpr int N = 4;
};
template <>
struct Vec16<bf16> {
  using V = bf16x8;
  static constexpr int N = 8;
};

// 16 bytes of every operand per thread step (all pointers 16-byte aligned); the n % N tail
// elements one per thread
template <typename T, int OP>
__global__ __launch_bounds__(256) void ew_vec_kernel(const T* a, const T* b, const T* c, const T* d, T* out,
                                                     int64_t n) {
  using V = typename Vec16<T>::V;
  constexpr int N = Vec16<T>::N;
  const int64_t ng = n / N, stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  for (int64_t g = t0; g < ng; g += stride) {
    const V va = ld_stream(reinterpret_cast<const V*>(a) + g);
    V vb = va, vc = va, vd = va, r;
    if (OP != EW_SILU) {
      vb = ld_stream(reinterpret_cast<const V*>(b) + g);
      vc = ld_stream(reinterpret_cast<const V*>(c) + g);
    }
    if (OP == EW_BIAS_GATED) vd = ld_stream(reinterpret_cast<const V*>(d) + g);
#pragma unroll
    for (int j = 0; j < N; ++j) r[j] = (T)ew_op<OP>((float)va[j], (float)vb[j], (float)vc[j], (float)vd[j]);
    st_stream(reinterpret_cast<V*>(out) + g, r);
  }
  for (int64_t i = ng * N + t0; i < n; i += stride) {
    const float vb = OP != EW_SILU ? ld<T>(b, i) : 0.f, vc = OP != EW_SILU ? ld<T>(c, i) : 0.f;
    const float vd = OP == EW_BIAS_GATED ? ld<T>(d, i) : 0.f;
    st<T>(out, i, ew_op<OP>(ld<T>(a, i), vb, vc, vd));
  }
}

unsigned ew_grid(int64_t n) {
  int64_t g = (n + 255) / 256;
  return (unsigned)(g > 8192 ? 8192 : (g < 1 ? 1 : g));
}

template <typename T, int OP>
void ew_dispatch(const void* a, const void* b, const void* c, const void* d, void* out, int64_t n, hipStream_t s) {
  const T *pa = (const T*)a, *pb = (const T*)b, *pc = (const T*)c, *pd = (const T*)d;
  if (oasis_aligned(16, pa, pb, pc, pd, (const T*)out))
    hipLaunchKernelGGL((ew_vec_kernel<T, OP>), dim3(ew_grid(n / Vec16<T>::N)), dim3(256), 0, s, pa, pb, pc, pd,
                       (T*)out, n);
  else
    hipLaunchKernelGGL((ew_kernel<T, OP>), dim3(ew_grid(n)), dim3(256), 0, s, pa, pb, pc, pd, (T*)out, n);
}

template <int OP>
int ew_launch(const void* a, const void* b, const void* c, const void* d, void* out, int64_t n, int dtype,
              oasis_stream_t stream, const char* what) {
  OASIS_REQUIRE(n >= 0, OASIS_ERR_SHAPE, "%s: negative n", what);
  if (n == 0) return OASIS_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == OASIS_F32) {
    ew_dispatch<float, OP>(a, b, c, d, out, n, s);
  } else if (dtype == OASIS_BF16) {
    ew_dispatch<bf16, OP>(a, b, c, d, out, n, s);
  } else {
    oasis::set_error("%s: unsupported dtype %d", what, dtype);
    return OASIS_ERR_DTYPE;
  }
  return oasis::check_launch(what);
}

__global__ void ddim_kernel(float* chunk, const float* v, int64_t n, DdimCoeffs k) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x)
    chunk[i] = ddim_step(chunk[i], v[i], k);
}

// latent row r = (h*2+p)*(2gw) + (w*2+q), col c  <-  chunk row h*gw+w, col (p*2+q)*C + c
__global__ void bridge_kernel(const float* chunk, float* lat, int gh, int gw, int C, int out_cols, float inv) {
  const int64_t n = (int64_t)gh * 2 * gw * 2 * out_cols;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int col = (int)(i % out_cols);
    const int64_t r = i / out_cols;
    float val = 0.f;
    if (col < C) {
      const int wq = (int)(r % (2 * gw)), hp = (int)(r / (2 * gw));
      const int h = hp >> 1, p = hp & 1, w = wq >> 1, q = wq & 1;
      val = chunk[((int64_t)h * gw + w) * (4 * C) + (p * 2 + q) * C + col] * inv;
    }
    lat[i] = val;
  }
}

// frame[c][hh*ps+pp][ww*ps+qq] = clamp(patches[hh*gw+ww][(c*ps+pp)*ps+qq])
__global__ void unpatchify_kernel(const float* patches, float* frame, int gh, int gw, int ps) {
  const int64_t H = (int64_t)gh * ps, W = (int64_t)gw * ps, n = 3 * H * W;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t x = i % W, y = (i / W) % H, c = i / (W * H);
    const int64_t hh = y / ps, pp = y % ps, ww = x / ps, qq = x % ps;
    const float v = patches[(hh * gw + ww) * (3 * ps * ps) + (c * ps + pp) * ps + qq];
    frame[i] = fminf(fmaxf(v, -1.0f), 1.0f);
  }
}

// Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as easy as 1, 2, 3",
// SC 2011): ten rounds of two 32 x 32 -> 64-bit products mixed with the key, the key bumped by
// the two Weyl constants between rounds. A counter-based generator: output i depends only on
// (key, counter), so every lane draws its own numbers with no state.
OASIS_DEV void philox4x32_10(uint32_t (&c)[4], uint32_t k0, uint32_t k1) {
  constexpr uint32_t M0 = 0xD2511F53u, M1 = 0xCD9E8D57u, W0 = 0x9E3779B9u, W1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint64_t p0 = (uint64_t)M0 * c[0], p1 = (uint64_t)M1 * c[2];
    const uint32_t hi0 = (uint32_t)(p0 >> 32), lo0 = (uint32_t)p0, hi1 = (uint32_t)(p1 >> 32), lo1 = (uint32_t)p1;
    const uint32_t n0 = hi1 ^ c[1] ^ k0, n2 = hi0 ^ c[3] ^ k1;
    c[0] = n0;
    c[1] = lo1;
    c[2] = n2;
    c[3] = lo0;
    k0 += W0;
    k1 += W1;
  }
}

// out[i] = clamp(N(0, 1) draw, -lim, lim) for i < n (and copy[i] the same when copy is set): one
// workgroup; draw i comes from Philox block (i / 4, *counter) under key (k0, k1) through the
// Box-Muller transform of its uniforms (2j, 2j+1) in (0, 1). *counter is then bumped, so a graph
// replaying this kernel draws fresh numbers every replay.
__global__ __launch_bounds__(256) void noise_kernel(float* __restrict__ out, float* __restrict__ copy, int64_t n,
                                                    uint32_t k0, uint32_t k1, uint32_t* __restrict__ counter,
                                                    float lim) {
  const uint32_t frame = counter[0];
  for (int64_t q = threadIdx.x; q * 4 < n; q += blockDim.x) {
    uint32_t x[4] = {(uint32_t)q, (uint32_t)(q >> 32), frame, 0u};
    philox4x32_10(x, k0, k1);
    float z[4];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      const float u1 = ((float)x[2 * j] + 0.5f) * 2.3283064365386963e-10f;  // (0, 1): 2^-32 steps
      const float u2 = ((float)x[2 * j + 1] + 0.5f) * 2.3283064365386963e-10f;
      const float r = sqrtf(-2.0f * logf(u1));
      float sn, cs;
      sincosf(6.283185307179586f * u2, &sn, &cs);
      z[2 * j] = r * cs;
      z[2 * j + 1] = r * sn;
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t i = 4 * q + j;
      if (i < n) {
        const float v = fminf(fmaxf(z[j], -lim), lim);
        out[i] = v;
        if (copy) copy[i] = v;
      }
    }
  }
  __syncthreads();  // every lane has read the counter
  if (threadIdx.x == 0) counter[0] = frame + 1u;
}

// CHW frame in [-1, 1] -> HWC in [0, 1]: out[(y*W + x)*C + c] = clamp((frame[(c*H + y)*W + x] + 1) / 2)
__global__ void frame_hwc_kernel(const float* __restrict__ frame, float* __restrict__ out, int C, int64_t HW) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < HW; i += (int64_t)gridDim.x * blockDim.x)
    for (int c = 0; c < C; ++c) out[i * C + c] = fminf(fmaxf((frame[c * HW + i] + 1.0f) * 0.5f, 0.0f), 1.0f);
}

__global__ void temb_kernel(const float* t, int64_t R, int half, float* out) {
  const int64_t n = R * half;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (int64_t)gridDim.x * blockDim.x) {
    const int64_t r = i / half;
    const int k = (int)(i % half);
    const float f = expf(-9.210340371976184f * (float)k / (float)half);  // ln(10000)
    const float a = t[r] * f;
    out[r * 2 * half + k] = cosf(a);
    out[r * 2 * half + half + k] = sinf(a);
  }
}

// out[m, n] = b[n] + sum_k x[m, k] W(n, k); block = R rows (staged in LDS), threads over n:
// each thread reads its weight row once for R outputs. W is bf16 or fp32 (TW), all sums fp32.
// KMAJOR: W(n, k) = W[k * N + n] (consecutive threads read consecutive addresses); else W[n * K + k].
template <int R, typename TW, bool KMAJOR>
__global__ __launch_bounds__(256) void small_linear_kernel(const float* x, int64_t ldx, int K, const TW* W,
                                                           int N, const float* b, float* out, int64_t ld_out,
                                                           int64_t M) {
  __shared__ float xs[R][256];
  const int64_t m0 = (int64_t)blockIdx.y * R;
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  for (int i = threadIdx.x; i < R * K; i += blockDim.x) {
    const int r = i / K, k = i - r * K;
    xs[r][k] = m0 + r < M ? x[(m0 + r) * ldx + k] : 0.f;
  }
  __syncthreads();
  if (n >= N) return;
  const TW* w = W + (int64_t)n * K;
  float acc[R];
#pragma unroll
  for (int r = 0; r < R; ++r) acc[r] = b ? b[n] : 0.f;
  for (int k = 0; k < K; k += 8) {
    float wv[8];
    if constexpr (KMAJOR) {
#pragma unroll
      for (int j = 0; j < 8; ++j) wv[j] = (float)W[(int64_t)(k + j) * N + n];
    } else if constexpr (sizeof(TW) == 2) {
      unpack8(*reinterpret_cast<const bf16x8*>(w + k), wv);
    } else {
      const f32x4 lo = *reinterpret_cast<const f32x4*>(w + k), hi = *reinterpret_cast<const f32x4*>(w + k + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        wv[j] = lo[j];
        wv[4 + j] = hi[j];
      }
    }
#pragma unroll
    for (int r = 0; r < R; ++r)
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[r] = fmaf(xs[r][k + j], wv[j], acc[r]);
  }
#pragma unroll
  for (int r = 0; r < R; ++r)
    if (m0 + r < M) out[(m0 + r) * ld_out + n] = acc[r];
}

// reference surface: out[r, n] = sum_k c[k] w[k, n] + b[n] (w is [K, N]), rows r < out_rows.
__global__ void adaln_expand_kernel(const float* c, const bf16* w, const float* b, float* out, int K, int N,
                                    int64_t rows) {
  const int n = blockIdx.x * blockDim.x + threadIdx.x;
  if (n >= N) return;
  float acc = b ? b[n] : 0.f;
  for (int k = 0; k < K; ++k) acc += c[k] * bf2f(w[(int64_t)k * N + n]);
  for (int64_t r = 0; r < rows; ++r) out[r * N + n] = acc;
}

// Standalone RoPE + head split: one workgroup per row, one thread per 8 consecutive dims of one
// (q|k|v, head) of it, every operand moved as 16-byte vectors (the tables as two 4-float vectors).
template <typename T>
__device__ __forceinline__ void ld8(const T* p, float* v);
template <>
__device__ __forceinline__ void ld8<float>(const float* p, float* v) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p), b = *reinterpret_cast<const f32x4*>(p + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = a[j];
    v[4 + j] = b[j];
  }
}
template <>
__device__ __forceinline__ void ld8<bf16>(const bf16* p, float* v) {
  unpack8(*reinterpret_cast<const bf16x8*>(p), v);
}
template <typename T>
__device__ __forceinline__ void st8(T* p, const float* v);
template <>
__device__ __forceinline__ void st8<float>(float* p, const float* v) {
  st_stream(reinterpret_cast<f32x4*>(p), f32x4{v[0], v[1], v[2], v[3]});
  st_stream(reinterpret_cast<f32x4*>(p + 4), f32x4{v[4], v[5], v[6], v[7]});
}
template <>
__device__ __forceinline__ void st8<bf16>(bf16* p, const float* v) {
  st_stream(reinterpret_cast<bf16x8*>(p), pack8(v));
}

// A workgroup takes up to RPG rows that share one table position (rows
// (q * pos_mod + pos) * pos_div + rem): thread t owns column group c8 = 8t of Q, K and V, loads its
// 8 cos / sin values once for all of them, and issues the loads of all its rows before any store.
// QKV rows are read with streaming loads and Q, K, V written with streaming stores (each byte is
// touched once). The elementwise kernels above stream their operands the same way. One row per
// workgroup times fastest (4608 rows: 12.9 us against 12.9 with 2 rows, 13.4 with 4 and 17.5 with
// 8; 288 rows: 2.55 against 2.86 and 3.11 us): more, smaller workgroups spread the rows' loads and
// stores over more waves.
constexpr int RPG = 1;

template <typename T, int MODE>
__global__ __launch_bounds__(256) void rope_layout_kernel(const T* qkv, int64_t ldq, const float* cs, const float* sn,
                                                          int64_t tab_ld, int64_t tab_hs, int64_t pos_div,
                                                          int64_t pos_mod, T* qo, T* ko, T* vo, int64_t rows,
                                                          int64_t seq, int H) {
  const int D = H * 64;
  const int64_t pos = blockIdx.x;
  int64_t row[RPG];
#pragma unroll
  for (int i = 0; i < RPG; ++i) {  // the j-th row of this position, j = blockIdx.y * RPG + i (rows: -1 past the end)
    // 32-bit divisions (the host checks that j, pos_div, seq and rows are below 2^31)
    const uint32_t j = blockIdx.y * RPG + i;
    const uint32_t q = j / (uint32_t)pos_div, rem = j - q * (uint32_t)pos_div;
    const int64_t r = ((int64_t)q * pos_mod + pos) * pos_div + rem;
    row[i] = r < rows ? r : -1;
  }
  if (row[0] < 0) return;  // no row of this workgroup exists (nor does its table row, necessarily)
  // 8 values of T as raw 16-byte vectors (one for bf16, two for fp32), converted at use
  constexpr int NV = sizeof(T) * 8 / 16;
  for (int t = threadIdx.x; t < D / 8; t += blockDim.x) {
    const int c8 = t * 8, h = c8 >> 6, d0 = c8 & 63;
    float c[8], s[8];
    i32x4 raw[RPG][3][NV];
    ld8<float>(cs + pos * tab_ld + h * tab_hs + d0, c);
    ld8<float>(sn + pos * tab_ld + h * tab_hs + d0, s);
#pragma unroll
    for (int i = 0; i < RPG; ++i)
      if (row[i] >= 0) {
#pragma unroll
        for (int w = 0; w < 3; ++w)
#pragma unroll
          for (int u = 0; u < NV; ++u)
            raw[i][w][u] = ld_stream(reinterpret_cast<const i32x4*>(qkv + row[i] * ldq + w * D + c8) + u);
      }
#pragma unroll
    for (int i = 0; i < RPG; ++i) {
      if (row[i] < 0) break;
      const uint32_t f = (uint32_t)row[i] / (uint32_t)seq, p = (uint32_t)row[i] - f * (uint32_t)seq;
      float v[3][8], r[2][8];
#pragma unroll
      for (int w = 0; w < 3; ++w) ld8<T>(reinterpret_cast<const T*>(raw[i][w]), v[w]);
#pragma unroll
      for (int w = 0; w < 2; ++w)
#pragma unroll
        for (int e = 0; e < 8; ++e) r[w][e] = v[w][e] * c[e] + v[w][e ^ 1] * s[e];
      const int64_t off = MODE == 0 ? (((int64_t)f * H + h) * seq + p) * 64 + d0 : row[i] * D + c8;
      st8<T>(qo + off, r[0]);
      st8<T>(ko + off, r[1]);
      st8<T>(vo + off, v[2]);
    }
  }
}

}  // namespace

extern "C" int oasis_silu(const void* x, void* out, int64_t n, int dtype, oasis_stream_t stream) {
  OASIS_REQUIRE(x && out, OASIS_ERR_NULL, "silu: null pointer");
  return ew_launch<EW_SILU>(x, nullptr, nullptr, nullptr, out, n, dtype, stream, "silu");
}

extern "C" int oasis_adaln_modulate(const void* x, const void* shift, const void* scale, void* out, int64_t n,
                                    int dtype, oasis_stream_t stream) {
  OASIS_REQUIRE(x && shift && scale && out, OASIS_ERR_NULL, "adaln_modulate: null pointer");
  return ew_launch<EW_MODULATE>(x, shift, scale, nullptr, out, n, dtype, stream, "adaln_modulate");
}

extern "C" int oasis_gated_residual(const void* residual, const void* x, const void* gate, void* out, int64_t n,
                                    int dtype, oasis_stream_t stream) {
  OASIS_REQUIRE(residual && x && gate && out, OASIS_ERR_NULL, "gated_residual: null pointer");
  return ew_launch<EW_GATED>(residual, x, gate, nullptr, out, n, dtype, stream, "gated_residual");
}

extern "C" int oasis_bias_gated_residual(const void* residual, const void* x, const void* bias, const void* gate,
                                         void* out, int64_t n, int dtype, oasis_stream_t stream) {
  OASIS_REQUIRE(residual && x && bias && gate && out, OASIS_ERR_NULL, "bias_gated_residual: null pointer");
  return ew_launch<EW_BIAS_GATED>(residual, x, bias, gate, out, n, dtype, stream, "bias_gated_residual");
}

extern "C" int oasis_ddim_update(float* chunk, const float* v, int64_t n, float c0, float c1, float c2, float c3,
                                 float c4, float c5, oasis_stream_t stream) {
  OASIS_REQUIRE(chunk && v, OASIS_ERR_NULL, "ddim_update: null pointer");
  OASIS_REQUIRE(n >= 0, OASIS_ERR_SHAPE, "ddim_update: negative n");
  if (n == 0) return OASIS_OK;
  const DdimCoeffs k = {{c0, c1, c2, c3, c4, c5}};
  hipLaunchKernelGGL(ddim_kernel, dim3(ew_grid(n)), dim3(256), 0, static_cast<hipStream_t>(stream), chunk, v, n, k);
  return oasis::check_launch("ddim_update");
}

extern "C" int oasis_bridge(const float* chunk, float* latent, int64_t gh, int64_t gw, int64_t C, int64_t out_cols,
                            float inv_scale, oasis_stream_t stream) {
  OASIS_REQUIRE(chunk && latent, OASIS_ERR_NULL, "bridge: null pointer");
  OASIS_REQUIRE(gh > 0 && gw > 0 && C > 0 && out_cols >= C, OASIS_ERR_SHAPE, "bridge: bad shape");
  const int64_t n = gh * 2 * gw * 2 * out_cols;
  hipLaunchKernelGGL(bridge_kernel, dim3(ew_grid(n)), dim3(256), 0, static_cast<hipStream_t>(stream), chunk, latent,
                     (int)gh, (int)gw, (int)C, (int)out_cols, inv_scale);
  return oasis::check_launch("bridge");
}

extern "C" int oasis_vae_unpatchify(const float* patches, float* frame, int64_t gh, int64_t gw, int64_t ps,
                                    oasis_stream_t stream) {
  OASIS_REQUIRE(patches && frame, OASIS_ERR_NULL, "vae_unpatchify: null pointer");
  OASIS_REQUIRE(gh > 0 && gw > 0 && ps > 0, OASIS_ERR_SHAPE, "vae_unpatchify: bad shape");
  const int64_t n = 3 * gh * ps * gw * ps;
  hipLaunchKernelGGL(unpatchify_kernel, dim3(ew_grid(n)), dim3(256), 0, static_cast<hipStream_t>(stream), patches,
                     frame, (int)gh, (int)gw, (int)ps);
  return oasis::check_launch("vae_unpatchify");
}

extern "C" int oasis_noise_normal(float* out, float* copy, int64_t n, uint64_t seed, uint32_t* counter,
                                  float clamp_abs, oasis_stream_t stream) {
  OASIS_REQUIRE(out && counter, OASIS_ERR_NULL, "noise_normal: null pointer");
  OASIS_REQUIRE(n > 0 && n <= (1ll << 34), OASIS_ERR_SHAPE, "noise_normal: n must be in [1, 2^34]");
  OASIS_REQUIRE(clamp_abs > 0.0f, OASIS_ERR_ARG, "noise_normal: clamp_abs must be positive");
  hipLaunchKernelGGL(noise_kernel, dim3(1), dim3(256), 0, static_cast<hipStream_t>(stream), out, copy, n,
                     (uint32_t)seed, (uint32_t)(seed >> 32), counter, clamp_abs);
  return oasis::check_launch("noise_normal");
}

extern "C" int oasis_frame_hwc(const float* frame, float* out, int64_t C, int64_t H, int64_t W,
                               oasis_stream_t stream) {
  OASIS_REQUIRE(frame && out, OASIS_ERR_NULL, "frame_hwc: null pointer");
  OASIS_REQUIRE(C > 0 && C <= 16 && H > 0 && W > 0, OASIS_ERR_SHAPE, "frame_hwc: bad shape");
  const int64_t HW = H * W;
  hipLaunchKernelGGL(frame_hwc_kernel, dim3(ew_grid(HW)), dim3(256), 0, static_cast<hipStream_t>(stream), frame, out,
                     (int)C, HW);
  return oasis::check_launch("frame_hwc");
}

extern "C" int oasis_timestep_embedding(const float* t, int64_t R, int64_t dim, float* out, oasis_stream_t stream) {
  OASIS_REQUIRE(t && out, OASIS_ERR_NULL, "timestep_embedding: null pointer");
  OASIS_REQUIRE(R > 0 && dim > 0 && dim % 2 == 0, OASIS_ERR_SHAPE, "timestep_embedding: bad shape");
  hipLaunchKernelGGL(temb_kernel, dim3(ew_grid(R * dim / 2)), dim3(256), 0, static_cast<hipStream_t>(stream), t, R,
                     (int)(dim / 2), out);
  return oasis::check_launch("timestep_embedding");
}

extern "C" int oasis_small_linear(const float* x, int64_t ldx, int64_t M, int64_t K, const void* W, int w_dtype,
                                  int w_layout, int64_t N, const float* b, float* out, int64_t ld_out,
                                  oasis_stream_t stream) {
  OASIS_REQUIRE(x && W && out, OASIS_ERR_NULL, "small_linear: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, W), OASIS_ERR_ARG, "small_linear: W must be 16-byte aligned");
  OASIS_REQUIRE(M > 0 && N > 0 && K > 0 && K <= 256 && K % 8 == 0 && ldx >= K && ld_out >= N, OASIS_ERR_SHAPE,
                "small_linear: need 0 < K <= 256, K % 8 == 0");
  OASIS_REQUIRE(M <= 65535 * 16, OASIS_ERR_SHAPE, "small_linear: M too large");
  OASIS_REQUIRE(w_dtype == OASIS_F32 || w_dtype == OASIS_BF16, OASIS_ERR_DTYPE, "small_linear: unsupported w_dtype %d",
                w_dtype);
  OASIS_REQUIRE(w_layout == 0 || w_layout == 1, OASIS_ERR_ARG, "small_linear: w_layout must be 0 ([N,K]) or 1 ([K,N])");
  const dim3 blk(256);
  const unsigned nb = (unsigned)((N + 255) / 256);
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bool big = M >= 2048;
  const dim3 grid(nb, (unsigned)(big ? (M + 15) / 16 : (M + 3) / 4));
  OASIS_REQUIRE(grid.y <= 65535, OASIS_ERR_SHAPE, "small_linear: M too large");
#define OASIS_SL(RV, TW, KM) \
  hipLaunchKernelGGL((small_linear_kernel<RV, TW, KM>), grid, blk, 0, s, x, ldx, (int)K, static_cast<const TW*>(W), \
                     (int)N, b, out, ld_out, M)
#define OASIS_SL2(TW, KM) \
  if (big) OASIS_SL(16, TW, KM); else OASIS_SL(4, TW, KM)
  if (w_dtype == OASIS_BF16) {
    if (w_layout) { OASIS_SL2(bf16, true); } else { OASIS_SL2(bf16, false); }
  } else {
    if (w_layout) { OASIS_SL2(float, true); } else { OASIS_SL2(float, false); }
  }
#undef OASIS_SL2
#undef OASIS_SL
  return oasis::check_launch("small_linear");
}

extern "C" int oasis_adaln_matmul_expand(const float* silu_cond, const void* w, const float* b, float* out,
                                         int64_t K, int64_t N, int64_t out_rows, oasis_stream_t stream) {
  OASIS_REQUIRE(silu_cond && w && out, OASIS_ERR_NULL, "adaln_matmul_expand: null pointer");
  OASIS_REQUIRE(K > 0 && N > 0 && out_rows > 0, OASIS_ERR_SHAPE, "adaln_matmul_expand: bad shape");
  hipLaunchKernelGGL(adaln_expand_kernel, dim3((unsigned)((N + 255) / 256)), dim3(256), 0,
                     static_cast<hipStream_t>(stream), silu_cond, static_cast<const bf16*>(w), b, out, (int)K, (int)N,
                     out_rows);
  return oasis::check_launch("adaln_matmul_expand");
}

extern "C" int oasis_rope_layout(const void* qkv, int64_t ld_qkv, const float* cos, const float* sinp, int64_t tab_ld,
                                 int64_t tab_head_stride, int64_t pos_div, int64_t pos_mod, void* q_out, void* k_out,
                                 void* v_out, int64_t rows, int64_t seq, int64_t n_heads, int64_t head_dim, int mode,
                                 int dtype, oasis_stream_t stream) {
  OASIS_REQUIRE(qkv && cos && sinp && q_out && k_out && v_out, OASIS_ERR_NULL, "rope_layout: null pointer");
  OASIS_REQUIRE(head_dim == 64, OASIS_ERR_SHAPE, "rope_layout: head_dim must be 64");
  OASIS_REQUIRE(rows > 0 && seq > 0 && n_heads > 0 && ld_qkv >= 3 * n_heads * 64 && pos_div > 0 && pos_mod > 0,
                OASIS_ERR_SHAPE, "rope_layout: bad shape");
  OASIS_REQUIRE(mode == 0 || mode == 1, OASIS_ERR_ARG, "rope_layout: mode must be 0 or 1");
  OASIS_REQUIRE(mode == 1 || rows % seq == 0, OASIS_ERR_SHAPE, "rope_layout: rows must be a multiple of seq");
  const size_t esz = dtype == OASIS_F32 ? 4 : 2;
  OASIS_REQUIRE(oasis_aligned(16, qkv, q_out, k_out, v_out, cos, sinp) && (ld_qkv * esz) % 16 == 0 && tab_ld % 4 == 0 &&
                    tab_head_stride % 4 == 0,
                OASIS_ERR_ARG, "rope_layout: pointers, ld_qkv rows and table strides must be 16-byte aligned");
  OASIS_REQUIRE(rows < (1ll << 31) && pos_div < (1ll << 31) && seq < (1ll << 31), OASIS_ERR_SHAPE,
                "rope_layout: rows, pos_div and seq must be below 2^31");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // rows per table position, then workgroups of up to RPG of them per position
  const int64_t per_pos = ((rows + pos_mod * pos_div - 1) / (pos_mod * pos_div)) * pos_div;
  const int64_t groups = (per_pos + RPG - 1) / RPG;
  OASIS_REQUIRE(pos_mod < (1ll << 31) && groups <= 65535, OASIS_ERR_SHAPE, "rope_layout: too many rows per position");
  const dim3 grid((unsigned)pos_mod, (unsigned)groups);
  const int threads = (int)std::min<int64_t>(256, n_heads * 8);
#define OASIS_ROPE(TT, MM)                                                                                        \
  hipLaunchKernelGGL((rope_layout_kernel<TT, MM>), grid, dim3(threads), 0, s, (const TT*)qkv, ld_qkv, cos, sinp, tab_ld, \
                     tab_head_stride, pos_div, pos_mod, (TT*)q_out, (TT*)k_out, (TT*)v_out, rows, seq, (int)n_heads)
  if (dtype == OASIS_F32) {
    if (mode == 0) OASIS_ROPE(float, 0); else OASIS_ROPE(float, 1);
  } else if (dtype == OASIS_BF16) {
    if (mode == 0) OASIS_ROPE(bf16, 0); else OASIS_ROPE(bf16, 1);
  } else {
    oasis::set_error("rope_layout: unsupported dtype %d", dtype);
    return OASIS_ERR_DTYPE;
  }
#undef OASIS_ROPE
  return oasis::check_launch("rope_layout");
}
