// Skinny GEMM for up to 32 conditioning rows per pass (adaLN projections and the conditioning
// MLP): out[r, n] = act_out(sum_k act_in(x[r, k]) W[n, k] + b[n]).
//
// This is pure weight streaming (the adaLN matrices of all sub-blocks are 406 MB of
// bf16 per DiT step against ~0.8 GFLOP), so the kernel is shaped around HBM:
//   - W rows are read as 16-byte vectors straight into MFMA A operands
//     (v_mfma_f32_16x16x32_bf16, 16 weight rows x 32 k per instruction), two k-steps
//     per 128-byte cache line and several k-steps in flight per wave;
//   - x (16 rows per row group, one or two groups) is staged once per workgroup in LDS as a
//     bf16 hi + lo pair,
//     x = hi + lo to ~16 mantissa bits, and both halves go through the MFMA, so the
//     result keeps fp32-level accuracy although the MFMA inputs are bf16;
//   - every wave walks its own 16-row weight tiles, so each byte of W is read once.
#include <algorithm>

#include "oasis_common.h"

namespace {

constexpr int KSTEP = 64;   // k per pipeline step (two MFMAs)
constexpr int UNROLL = 4;   // pipeline steps whose loads are issued together

template <int RG>
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x, int64_t ldx, int R,
                                                   const bf16* __restrict__ W, int N, int K,
                                                   const float* __restrict__ b, float* __restrict__ out,
                                                   int64_t ld_out, int act_in, int act_out, int accumulate) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  const int pitch = K + 8;  // bf16 elements per LDS row
  bf16* xh = reinterpret_cast<bf16*>(smem_raw);
  bf16* xl = xh + R * pitch;
  for (int i = threadIdx.x; i < R * K; i += blockDim.x) {
    const int r = i / K, kk = i - r * K;
    float val = x[(int64_t)r * ldx + kk];
    if (act_in == OASIS_ACT_SILU) val = silu(val);
    const bf16 hi = f2bf(val);
    xh[r * pitch + kk] = hi;
    xl[r * pitch + kk] = f2bf(val - bf2f(hi));
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, lr = lane & 15, g = lane >> 4;
  const int waves_total = gridDim.x * (blockDim.x >> 6);
  const int tiles = N >> 4;
  // row group q covers conditioning rows 16q..16q+15; lanes whose row is >= R feed zeros to the
  // MFMA B operand
  bool live[RG];
  const bf16* xhp[RG];
  const bf16* xlp[RG];
#pragma unroll
  for (int q = 0; q < RG; ++q) {
    live[q] = 16 * q + lr < R;
    xhp[q] = xh + (live[q] ? 16 * q + lr : 0) * pitch + g * 8;
    xlp[q] = xl + (live[q] ? 16 * q + lr : 0) * pitch + g * 8;
  }
  bf16x8 zero;
#pragma unroll
  for (int j = 0; j < 8; ++j) zero[j] = f2bf(0.f);
  for (int tile = blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); tile < tiles; tile += waves_total) {
    const bf16* wp = W + ((int64_t)tile * 16 + lr) * K + g * 8;
    f32x4 acc[RG];
#pragma unroll
    for (int q = 0; q < RG; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = 0; k0 < K; k0 += KSTEP * UNROLL) {
      bf16x8 w[UNROLL][2];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int kk = k0 + u * KSTEP;
        if (kk < K) {
          w[u][0] = *reinterpret_cast<const bf16x8*>(wp + kk);
          w[u][1] = *reinterpret_cast<const bf16x8*>(wp + kk + 32);
        }
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int kk = k0 + u * KSTEP;
        if (kk < K) {
#pragma unroll
          for (int q = 0; q < RG; ++q) {
            const bf16x8 h0 = live[q] ? *reinterpret_cast<const bf16x8*>(xhp[q] + kk) : zero;
            const bf16x8 l0 = live[q] ? *reinterpret_cast<const bf16x8*>(xlp[q] + kk) : zero;
            const bf16x8 h1 = live[q] ? *reinterpret_cast<const bf16x8*>(xhp[q] + kk + 32) : zero;
            const bf16x8 l1 = live[q] ? *reinterpret_cast<const bf16x8*>(xlp[q] + kk + 32) : zero;
            acc[q] = mfma16(w[u][0], h0, acc[q]);
            acc[q] = mfma16(w[u][0], l0, acc[q]);
            acc[q] = mfma16(w[u][1], h1, acc[q]);
            acc[q] = mfma16(w[u][1], l1, acc[q]);
          }
        }
      }
    }
    // acc[q][i] = out[r = 16q + lr][n = tile*16 + 4g + i]
#pragma unroll
    for (int q = 0; q < RG; ++q) {
      if (!live[q]) continue;
      const int n0 = tile * 16 + 4 * g;
      float v[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        v[i] = acc[q][i] + (b ? b[n0 + i] : 0.f);
        if (act_out == OASIS_ACT_SILU) v[i] = silu(v[i]);
      }
      float* o = out + (int64_t)(16 * q + lr) * ld_out + n0;
      if (accumulate) {
#pragma unroll
        for (int i = 0; i < 4; ++i) v[i] += o[i];
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = v[i];
    }
  }
}

}  // namespace

extern "C" int oasis_gemv_bf16(const float* x, int64_t ldx, int64_t R, const void* W, int64_t N, int64_t K,
                               const float* b, float* out, int64_t ld_out, int act_in, int act_out, int accumulate,
                               oasis_stream_t stream) {
  OASIS_REQUIRE(x && W && out, OASIS_ERR_NULL, "gemv: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, W), OASIS_ERR_ARG, "gemv: W must be 16-byte aligned");
  OASIS_REQUIRE(R > 0 && R <= 1024, OASIS_ERR_SHAPE, "gemv: R=%lld must be in [1, 1024]", (long long)R);
  OASIS_REQUIRE(K > 0 && K % KSTEP == 0 && K <= 2048, OASIS_ERR_SHAPE, "gemv: K=%lld must be a multiple of 64, <= 2048",
                (long long)K);
  OASIS_REQUIRE(N > 0 && N % 16 == 0 && N < (1ll << 31), OASIS_ERR_SHAPE, "gemv: N=%lld must be a multiple of 16",
                (long long)N);
  OASIS_REQUIRE(ldx >= K && ld_out >= N, OASIS_ERR_SHAPE, "gemv: ldx/ld_out too small");
  OASIS_REQUIRE((act_in == OASIS_ACT_NONE || act_in == OASIS_ACT_SILU) &&
                    (act_out == OASIS_ACT_NONE || act_out == OASIS_ACT_SILU),
                OASIS_ERR_ARG, "gemv: bad activation");
  // one pass over W per 32 rows (two 16-row groups) while x fits in LDS, else per 16 rows
  const int per_pass = 2 * 32 * (K + 8) * (int64_t)sizeof(bf16) <= 160 * 1024 ? 32 : 16;
  for (int64_t r0 = per_pass; r0 < R; r0 += per_pass) {
    const int rc = oasis_gemv_bf16(x + r0 * ldx, ldx, R - r0 < per_pass ? R - r0 : per_pass, W, N, K, b,
                                   out + r0 * ld_out, ld_out, act_in, act_out, accumulate, stream);
    if (rc != OASIS_OK) return rc;
  }
  if (R > per_pass) R = per_pass;
  const int tiles = (int)(N / 16);
  const size_t smem = 2 * (size_t)R * (size_t)(K + 8) * sizeof(bf16);
  // every workgroup stages x once, so the grid stays at about two waves of resident
  // workgroups (LDS-limited) and each wave walks many weight tiles
  const int resident = (int)std::min<size_t>(8, (160 * 1024) / std::max<size_t>(smem, 1));
  int blocks = (tiles + 3) / 4;
  blocks = std::min(std::min(blocks, 2048), std::max(1, resident) * 256 * 2);
  const void* fn = R > 16 ? reinterpret_cast<const void*>(&gemv_kernel<2>) : reinterpret_cast<const void*>(&gemv_kernel<1>);
  if (smem > 65536) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) {
      oasis::set_error("gemv: cannot reserve %zu bytes of LDS: %s", smem, hipGetErrorString(e));
      return OASIS_ERR_LAUNCH;
    }
  }
  if (R > 16)
    hipLaunchKernelGGL(gemv_kernel<2>, dim3(blocks), dim3(256), smem, static_cast<hipStream_t>(stream), x, ldx, (int)R,
                       static_cast<const bf16*>(W), (int)N, (int)K, b, out, ld_out, act_in, act_out, accumulate);
  else
    hipLaunchKernelGGL(gemv_kernel<1>, dim3(blocks), dim3(256), smem, static_cast<hipStream_t>(stream), x, ldx, (int)R,
                       static_cast<const bf16*>(W), (int)N, (int)K, b, out, ld_out, act_in, act_out, accumulate);
  return oasis::check_launch("gemv");
}
