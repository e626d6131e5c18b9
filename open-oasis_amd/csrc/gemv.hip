// Skinny GEMM for up to 32 conditioning rows per pass (adaLN projections and the conditioning
// MLP): out[r, n] = act_out(sum_k act_in(x[r, k]) W[n, k] + b[n]).
//
// This is pure weight streaming (the adaLN matrices of all sub-blocks are 406 MB of
// bf16 per DiT step against ~0.8 GFLOP), so the kernel is shaped around HBM:
//   - W rows are read as 16-byte streaming vectors straight into MFMA A operands
//     (v_mfma_f32_16x16x32_bf16, 16 weight rows x 32 k per instruction), two k-steps
//     per 128-byte cache line and several k-steps in flight per wave;
//   - x (16 rows per row group, one or two groups) is staged once per workgroup in LDS as a
//     bf16 hi + lo pair,
//     x = hi + lo to ~16 mantissa bits, and both halves go through the MFMA, so the
//     result keeps fp32-level accuracy although the MFMA inputs are bf16;
//   - every wave walks its own 16-row weight tiles, so each byte of W is read once;
//   - small N (the conditioning MLP's 1024 outputs): the four waves of a workgroup share
//     each tile, one K quarter each, and add their partial sums through LDS, so that 4x
//     more waves stream the matrix and each one's dependent load chain is 4x shorter.
#include <algorithm>

#include "oasis_common.h"

namespace {

constexpr int KSTEP = 64;   // k per pipeline step (two MFMAs)
// pipeline steps whose loads are issued together (gemv_tiles' UNROLL): 4 with one 16-row group of
// x; 8 with two, whose staged x (132 KB at 32 rows) leaves one workgroup per CU, so each wave keeps
// more in flight (the config-4 adaLN pass over 32 rows 180 -> 171 us)

// TILED: W in 16-row MFMA tile order (for tile t and 32-wide K step s, the 64 lanes' 16-byte
// pieces back to back, lane l holding row 16t + (l & 15), columns 32s + 8(l >> 4) .. +7), so a
// wave's load instruction reads 1 KB contiguous; else row-major [N, K].
// block / nblocks: this workgroup's index among the nblocks that share the tiles
template <int RG, int KS, bool TILED, int UNROLL = RG == 1 ? 4 : 8>
__device__ __forceinline__ void gemv_tiles(const float* __restrict__ x, int64_t ldx, int R, const bf16* __restrict__ W,
                                           int N, int K, const float* __restrict__ b, float* __restrict__ out,
                                           int64_t ld_out, int act_in, int act_out, int accumulate, int block,
                                           int nblocks) {
  static_assert(KS == 1 || KS == 2 || KS == 4, "waves per tile");
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  const int pitch = K + 8;  // bf16 elements per LDS row
  bf16* xh = reinterpret_cast<bf16*>(smem_raw);
  bf16* xl = xh + R * pitch;
  // KS > 1: partial sums of the waves sharing a tile, after the x rows (16-byte aligned)
  f32x4* red = reinterpret_cast<f32x4*>(smem_raw + ((2 * R * pitch * sizeof(bf16) + 15) & ~size_t(15)));
  for (int i = threadIdx.x; i < R * K; i += blockDim.x) {
    const int r = i / K, kk = i - r * K;
    float val = x[(int64_t)r * ldx + kk];
    if (act_in == OASIS_ACT_SILU) val = silu(val);
    const bf16 hi = f2bf(val);
    xh[r * pitch + kk] = hi;
    xl[r * pitch + kk] = f2bf(val - bf2f(hi));
  }
  __syncthreads();

  const int lane = threadIdx.x & 63, lr = lane & 15, g = lane >> 4, wave = threadIdx.x >> 6;
  // KS waves per tile, each over K / KS (a multiple of KSTEP)
  const int tiles_per_block = (blockDim.x >> 6) / KS;
  const int waves_total = nblocks * tiles_per_block;
  const int tiles = N >> 4;
  const int kpart = wave % KS, kq = K / KS;
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
  // KS > 1: every wave of the workgroup runs the same number of iterations (one tile per
  // workgroup per iteration), so the barriers of the reduction below are uniform
  for (int tile0 = block * tiles_per_block; tile0 < tiles; tile0 += waves_total) {
    const int tile = tile0 + wave / KS;
    const bool has_tile = tile < tiles;
    if (KS == 1 && !has_tile) continue;  // no barriers to keep in step with
    const int tl = has_tile ? tile : 0;
    // row-major: row 16 tl + lr, columns 8g + kk; tiled: step kk / 32 of tile tl at 512 elements each
    const bf16* wp = TILED ? W + ((int64_t)tl * (K / 32) * 64 + lane) * 8 : W + ((int64_t)tl * 16 + lr) * K + g * 8;
    f32x4 acc[RG];
#pragma unroll
    for (int q = 0; q < RG; ++q) acc[q] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int kend = (kpart + 1) * kq;
    for (int k0 = kpart * kq; k0 < kend; k0 += KSTEP * UNROLL) {
      bf16x8 w[UNROLL][2];
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int kk = k0 + u * KSTEP;
        if (kk < kend) {
          const bf16* p0 = TILED ? wp + (kk / 32) * 512 : wp + kk;
          const bf16* p1 = TILED ? p0 + 512 : wp + kk + 32;
          w[u][0] = ld_stream(reinterpret_cast<const bf16x8*>(p0));
          w[u][1] = ld_stream(reinterpret_cast<const bf16x8*>(p1));
        }
      }
#pragma unroll
      for (int u = 0; u < UNROLL; ++u) {
        const int kk = k0 + u * KSTEP;
        if (kk < kend) {
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
    if (KS > 1) {  // wave kpart 0 of each tile adds the other K parts
#pragma unroll
      for (int q = 0; q < RG; ++q) red[(wave * RG + q) * 64 + lane] = acc[q];
      __syncthreads();
      if (kpart == 0) {
#pragma unroll
        for (int p = 1; p < KS; ++p)
#pragma unroll
          for (int q = 0; q < RG; ++q) acc[q] += red[((wave + p) * RG + q) * 64 + lane];
      }
      __syncthreads();  // the slots are rewritten by the next iteration
      if (kpart != 0) continue;
    }
    if (!has_tile) continue;
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

template <int RG, int KS, bool TILED>
__global__ __launch_bounds__(256) void gemv_kernel(const float* __restrict__ x, int64_t ldx, int R,
                                                   const bf16* __restrict__ W, int N, int K,
                                                   const float* __restrict__ b, float* __restrict__ out,
                                                   int64_t ld_out, int act_in, int act_out, int accumulate) {
  gemv_tiles<RG, KS, TILED>(x, ldx, R, W, N, K, b, out, ld_out, act_in, act_out, accumulate, blockIdx.x, gridDim.x);
}

}  // namespace

namespace {

int gemv_bf16(const float* x, int64_t ldx, int64_t R, const void* W, int64_t N, int64_t K, const float* b,
              float* out, int64_t ld_out, int act_in, int act_out, int accumulate, bool tiled, oasis_stream_t stream) {
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
    const int rc = gemv_bf16(x + r0 * ldx, ldx, R - r0 < per_pass ? R - r0 : per_pass, W, N, K, b,
                             out + r0 * ld_out, ld_out, act_in, act_out, accumulate, tiled, stream);
    if (rc != OASIS_OK) return rc;
  }
  if (R > per_pass) R = per_pass;
  const int tiles = (int)(N / 16);
  // waves per tile: with fewer tiles than 2 per CU, the largest of 4, 2 that splits K into
  // whole 64-wide steps
  int ks = 1;
  if (tiles < 512) ks = (K / KSTEP) % 4 == 0 ? 4 : ((K / KSTEP) % 2 == 0 ? 2 : 1);
  const int rg = R > 16 ? 2 : 1;
  const size_t xbytes = 2 * (size_t)R * (size_t)(K + 8) * sizeof(bf16);
  const size_t smem = ks > 1 ? ((xbytes + 15) & ~size_t(15)) + (size_t)4 * rg * 64 * sizeof(f32x4) : xbytes;
  // every workgroup stages x once, so the grid stays at about two waves of resident
  // workgroups (LDS-limited) and each wave walks many weight tiles
  const int resident = (int)std::min<size_t>(8, (160 * 1024) / std::max<size_t>(smem, 1));
  const int per_block = 4 / ks;
  int blocks = (tiles + per_block - 1) / per_block;
  blocks = std::min(std::min(blocks, 2048), std::max(1, resident) * 256 * 2);
  const void* fn = nullptr;
#define OASIS_GEMV_FN(RGV, KSV)                                                                                   \
  if (rg == RGV && ks == KSV)                                                                                     \
  fn = tiled ? reinterpret_cast<const void*>(&gemv_kernel<RGV, KSV, true>)                                        \
             : reinterpret_cast<const void*>(&gemv_kernel<RGV, KSV, false>)
  OASIS_GEMV_FN(1, 1);
  OASIS_GEMV_FN(1, 2);
  OASIS_GEMV_FN(1, 4);
  OASIS_GEMV_FN(2, 1);
  OASIS_GEMV_FN(2, 2);
  OASIS_GEMV_FN(2, 4);
#undef OASIS_GEMV_FN
  if (smem > 65536) {
    const hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) {
      oasis::set_error("gemv: cannot reserve %zu bytes of LDS: %s", smem, hipGetErrorString(e));
      return OASIS_ERR_LAUNCH;
    }
  }
  hipStream_t s = static_cast<hipStream_t>(stream);
  const bf16* Wb = static_cast<const bf16*>(W);
  const int Ri = (int)R, Ni = (int)N, Ki = (int)K;
#define OASIS_GEMV_GO(RGV, KSV)                                                                                   \
  if (rg == RGV && ks == KSV) {                                                                                   \
    if (tiled)                                                                                                    \
      hipLaunchKernelGGL((gemv_kernel<RGV, KSV, true>), dim3(blocks), dim3(256), smem, s, x, ldx, Ri, Wb, Ni, Ki, \
                         b, out, ld_out, act_in, act_out, accumulate);                                            \
    else                                                                                                          \
      hipLaunchKernelGGL((gemv_kernel<RGV, KSV, false>), dim3(blocks), dim3(256), smem, s, x, ldx, Ri, Wb, Ni,    \
                         Ki, b, out, ld_out, act_in, act_out, accumulate);                                        \
  }
  OASIS_GEMV_GO(1, 1);
  OASIS_GEMV_GO(1, 2);
  OASIS_GEMV_GO(1, 4);
  OASIS_GEMV_GO(2, 1);
  OASIS_GEMV_GO(2, 2);
  OASIS_GEMV_GO(2, 4);
#undef OASIS_GEMV_GO
  return oasis::check_launch("gemv");
}

}  // namespace

extern "C" int oasis_gemv_bf16(const float* x, int64_t ldx, int64_t R, const void* W, int64_t N, int64_t K,
                               const float* b, float* out, int64_t ld_out, int act_in, int act_out, int accumulate,
                               oasis_stream_t stream) {
  return gemv_bf16(x, ldx, R, W, N, K, b, out, ld_out, act_in, act_out, accumulate, false, stream);
}

extern "C" int oasis_gemv_bf16_tiled(const float* x, int64_t ldx, int64_t R, const void* W, int64_t N, int64_t K,
                                     const float* b, float* out, int64_t ld_out, int act_in, int act_out,
                                     int accumulate, oasis_stream_t stream) {
  return gemv_bf16(x, ldx, R, W, N, K, b, out, ld_out, act_in, act_out, accumulate, true, stream);
}

// ---------------------------------------------------------------------------------------
// fp32 weights: out[r, n] (+)= act_out(sum_k act_in(x[r, k]) W[n, k] + b[n]), everything fp32
// (fp32 products and sums, no bf16 anywhere). For the projections the reference keeps in fp32:
// the conditioning MLP and action projection (computed on the host in fp32,
// oasis_inference.py:512-520,1406-1427) and the final layer's adaLN
// (oasis_inference.py:527-532,1499-1511).
//   - up to RP conditioning rows per pass are staged in LDS as fp32 (act_in applied once;
//     act_in == OASIS_ACT_TEMB: x holds one timestep per row and the staged row is its
//     sinusoidal embedding [cos(t f_i), sin(t f_i)], f_i = exp(-ln(10000) i / (K/2)));
//   - a wave streams NU weight rows at a time as 1 KB coalesced vectors (lane l owns k = 4l..4l+3
//     of every 256-wide K chunk), multiplies them against every staged row, and reduces each
//     (n, r) dot product across the wave;
//   - every W byte is read once per pass.
constexpr int F32_RP = 8;    // conditioning rows per pass
constexpr int F32_NU = 2;    // weight rows per wave
constexpr int F32_CH = 4;    // 256-wide K chunks of a weight row held in registers at once

// Every wave owns F32_NU weight rows and issues the loads of their first 1024 columns before the
// workgroup stages x, so the HBM latency overlaps the staging; longer rows take further groups of
// 1024 columns. The multiplied row can be two inputs side by side: columns [0, K1) from x and
// [K1, K) from x2 (K1 = K without a second input).
__device__ __forceinline__ void gemv_f32_rows(const float* __restrict__ x, int64_t ldx, int K1,
                                              const float* __restrict__ x2, int64_t ldx2, int R,
                                              const float* __restrict__ W, int N, int K,
                                              const float* __restrict__ b, float* __restrict__ out, int64_t ld_out,
                                              int act_in, int act_out, int accumulate, int block) {
  extern __shared__ __attribute__((aligned(16))) char smem_raw[];
  float* xs = reinterpret_cast<float*>(smem_raw);  // [R][K], R <= F32_RP
  const int lane = threadIdx.x & 63;
  const int64_t n0 = ((int64_t)block * (blockDim.x >> 6) + (threadIdx.x >> 6)) * F32_NU;
  auto load_group = [&](int kb, f32x4 (&w)[F32_NU][F32_CH]) {
#pragma unroll
    for (int u = 0; u < F32_NU; ++u)
#pragma unroll
      for (int c = 0; c < F32_CH; ++c) {
        const int k = kb + c * 256 + lane * 4;
        w[u][c] = (n0 + u < N && k < K) ? *reinterpret_cast<const f32x4*>(W + (n0 + u) * K + k)
                                        : f32x4{0.f, 0.f, 0.f, 0.f};
      }
  };
  f32x4 w[F32_NU][F32_CH];
  load_group(0, w);
  // stage the R live rows (rows >= R are never read): 16-byte pieces, 4 per thread in flight
  const int k4 = K / 4, nvec = R * k4;
  for (int i0 = threadIdx.x; i0 < nvec; i0 += 4 * blockDim.x) {
    f32x4 v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j * blockDim.x;
      if (i >= nvec) break;
      const int r = i / k4, kk = 4 * (i - r * k4);
      if (act_in == OASIS_ACT_TEMB) {
        const float t = x[(int64_t)r * ldx];
        const int half = K / 2;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const int kj = kk + e, jj = kj < half ? kj : kj - half;
          const float a = t * expf(-9.210340371976184f * (float)jj / (float)half);  // ln(10000)
          v[j][e] = kj < half ? cosf(a) : sinf(a);
        }
      } else if (kk < K1) {
        v[j] = *reinterpret_cast<const f32x4*>(x + (int64_t)r * ldx + kk);
      } else {
        v[j] = *reinterpret_cast<const f32x4*>(x2 + (int64_t)r * ldx2 + (kk - K1));
      }
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int i = i0 + j * blockDim.x;
      if (i >= nvec) break;
      const int r = i / k4, kk = 4 * (i - r * k4);
      if (act_in == OASIS_ACT_SILU) {
#pragma unroll
        for (int e = 0; e < 4; ++e) v[j][e] = silu(v[j][e]);
      }
      *reinterpret_cast<f32x4*>(xs + r * K + kk) = v[j];
    }
  }
  __syncthreads();
  if (n0 >= N) return;  // after the only barrier
  float acc[F32_NU][F32_RP];
#pragma unroll
  for (int u = 0; u < F32_NU; ++u)
#pragma unroll
    for (int r = 0; r < F32_RP; ++r) acc[u][r] = 0.f;
  for (int kb = 0; kb < K; kb += 256 * F32_CH) {
    if (kb > 0) load_group(kb, w);
#pragma unroll
    for (int c = 0; c < F32_CH; ++c) {
      const int k = kb + c * 256 + lane * 4;
      if (k >= K) break;
#pragma unroll
      for (int r = 0; r < F32_RP; ++r) {
        if (r >= R) break;
        const f32x4 xv = *reinterpret_cast<const f32x4*>(xs + r * K + k);
#pragma unroll
        for (int u = 0; u < F32_NU; ++u)
          acc[u][r] = fmaf(w[u][c][3], xv[3], fmaf(w[u][c][2], xv[2], fmaf(w[u][c][1], xv[1],
                      fmaf(w[u][c][0], xv[0], acc[u][r]))));
      }
    }
  }
#pragma unroll
  for (int u = 0; u < F32_NU; ++u) {
#pragma unroll
    for (int r = 0; r < F32_RP; ++r) {
      if (r >= R) break;
      const float s = wave_sum(acc[u][r]);
      const int64_t n = n0 + u;
      if (lane == r && n < N) {
        float v = s + (b ? b[n] : 0.f);
        if (act_out == OASIS_ACT_SILU) v = silu(v);
        float* o = out + (int64_t)r * ld_out + n;
        *o = accumulate ? *o + v : v;
      }
    }
  }
}

__global__ __launch_bounds__(256) void gemv_f32_kernel(const float* __restrict__ x, int64_t ldx, int K1,
                                                       const float* __restrict__ x2, int64_t ldx2, int R,
                                                       const float* __restrict__ W, int N, int K,
                                                       const float* __restrict__ b, float* __restrict__ out,
                                                       int64_t ld_out, int act_in, int act_out, int accumulate) {
  gemv_f32_rows(x, ldx, K1, x2, ldx2, R, W, N, K, b, out, ld_out, act_in, act_out, accumulate, blockIdx.x);
}

// The two adaLN projections of a step's conditioning rows in one launch: workgroups [0, nb32) run
// the final layer's fp32 rows (gemv_f32_rows), the rest the sub-blocks' bf16 rows in MFMA tile
// order (gemv_tiles, one wave per 16-row tile). Both read the same rows x (SiLU applied), write
// into one output with row stride ld_out, and stage at most R * (K + 8) * 4 bytes of LDS.
__global__ __launch_bounds__(256) void gemv_adaln_pair_kernel(const float* __restrict__ x, int64_t ldx, int R,
                                                              const bf16* __restrict__ W16, int N16,
                                                              const float* __restrict__ b16, float* __restrict__ out16,
                                                              const float* __restrict__ W32, int N32,
                                                              const float* __restrict__ b32, float* __restrict__ out32,
                                                              int K, int64_t ld_out, int nb32) {
  if ((int)blockIdx.x < nb32)
    gemv_f32_rows(x, ldx, K, nullptr, 0, R, W32, N32, K, b32, out32, ld_out, OASIS_ACT_SILU, OASIS_ACT_NONE, 0,
                  blockIdx.x);
  else
    gemv_tiles<1, 1, true>(x, ldx, R, W16, N16, K, b16, out16, ld_out, OASIS_ACT_SILU, OASIS_ACT_NONE, 0,
                           blockIdx.x - nb32, gridDim.x - nb32);
}

namespace oasis {

// out16[r, :N16] = W16 silu(x_r) + b16 (bf16 weights in 16-row tile order) and
// out32[r, :N32] = W32 silu(x_r) + b32 (fp32 weights) for R <= 8 rows in one launch. Returns 1
// without launching when the shapes are outside what the pair kernel covers.
int gemv_adaln_pair(const float* x, int64_t ldx, int64_t R, const void* W16, int64_t N16, const float* b16,
                    float* out16, const float* W32, int64_t N32, const float* b32, float* out32, int64_t K,
                    int64_t ld_out, hipStream_t s) {
  if (!x || !W16 || !W32 || !out16 || !out32 || !oasis_aligned(16, W16, W32, x) || R < 1 || R > F32_RP ||
      K % KSTEP != 0 || K > 1024 || ldx < K || ldx % 4 != 0 || N16 % 16 != 0 || N16 / 16 < 512 ||
      N16 >= (1ll << 31) || N32 < 1 || N32 >= (1ll << 31) || ld_out < N16 || ld_out % 4 != 0)
    return 1;
  // the bf16 part's grid as gemv_bf16 sizes it for one row group and one wave per tile
  const size_t smem = 2 * (size_t)R * (size_t)(K + 8) * sizeof(bf16) > (size_t)R * K * sizeof(float)
                          ? 2 * (size_t)R * (size_t)(K + 8) * sizeof(bf16)
                          : (size_t)R * K * sizeof(float);
  const int resident = (int)std::min<size_t>(8, (160 * 1024) / smem);
  const int tiles = (int)(N16 / 16);
  const int nb16 = std::min(std::min((tiles + 3) / 4, 2048), std::max(1, resident) * 256 * 2);
  const int nb32 = (int)((N32 + 4 * F32_NU - 1) / (4 * F32_NU));
  hipLaunchKernelGGL(gemv_adaln_pair_kernel, dim3((unsigned)(nb32 + nb16)), dim3(256), smem, s, x, ldx, (int)R,
                     static_cast<const bf16*>(W16), (int)N16, b16, out16, W32, (int)N32, b32, out32, (int)K, ld_out,
                     nb32);
  return check_launch("gemv_adaln_pair");
}

int gemv_f32_cat(const float* x, int64_t ldx, int64_t K1, const float* x2, int64_t ldx2, int64_t R, const float* W,
                 int64_t N, int64_t K, const float* b, float* out, int64_t ld_out, int act_in, int act_out,
                 int accumulate, hipStream_t s) {
  OASIS_REQUIRE(x && W && out, OASIS_ERR_NULL, "gemv_f32: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, W), OASIS_ERR_ARG, "gemv_f32: W must be 16-byte aligned");
  OASIS_REQUIRE(R > 0 && R <= 1024, OASIS_ERR_SHAPE, "gemv_f32: R=%lld must be in [1, 1024]", (long long)R);
  OASIS_REQUIRE(K > 0 && K % 4 == 0 && K <= 4096, OASIS_ERR_SHAPE, "gemv_f32: K=%lld must be a multiple of 4, <= 4096",
                (long long)K);
  OASIS_REQUIRE(N > 0 && N < (1ll << 31), OASIS_ERR_SHAPE, "gemv_f32: bad N=%lld", (long long)N);
  OASIS_REQUIRE(K1 > 0 && K1 <= K && K1 % 4 == 0 && (K1 == K || (x2 && act_in != OASIS_ACT_TEMB)), OASIS_ERR_ARG,
                "gemv_f32: bad split of K between the two inputs");
  OASIS_REQUIRE((act_in == OASIS_ACT_TEMB ? ldx >= 1 : ldx >= K1 && ldx % 4 == 0) &&
                    (K1 == K || (ldx2 >= K - K1 && ldx2 % 4 == 0)) && ld_out >= N,
                OASIS_ERR_SHAPE, "gemv_f32: ldx/ld_out too small (x rows must be multiples of 4 floats)");
  OASIS_REQUIRE(act_in == OASIS_ACT_TEMB || oasis_aligned(16, x, x2), OASIS_ERR_ARG,
                "gemv_f32: x must be 16-byte aligned");
  OASIS_REQUIRE((act_in == OASIS_ACT_NONE || act_in == OASIS_ACT_SILU || act_in == OASIS_ACT_TEMB) &&
                    (act_out == OASIS_ACT_NONE || act_out == OASIS_ACT_SILU),
                OASIS_ERR_ARG, "gemv_f32: bad activation");
  const size_t smem = (size_t)F32_RP * K * sizeof(float);
  if (smem > 65536) {
    const hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(&gemv_f32_kernel),
                                             hipFuncAttributeMaxDynamicSharedMemorySize, (int)smem);
    if (e != hipSuccess) {
      oasis::set_error("gemv_f32: cannot reserve %zu bytes of LDS: %s", smem, hipGetErrorString(e));
      return OASIS_ERR_LAUNCH;
    }
  }
  // one wave per F32_NU weight rows
  const int64_t rows_per_block = 4 * F32_NU;
  const int64_t blocks = (N + rows_per_block - 1) / rows_per_block;
  for (int64_t r0 = 0; r0 < R; r0 += F32_RP) {
    const int rc = (int)std::min<int64_t>(F32_RP, R - r0);
    hipLaunchKernelGGL(gemv_f32_kernel, dim3((unsigned)blocks), dim3(256), smem, s, x + r0 * ldx, ldx, (int)K1,
                       x2 ? x2 + r0 * ldx2 : nullptr, ldx2, rc, W, (int)N, (int)K, b, out + r0 * ld_out, ld_out, act_in,
                       act_out, accumulate);
    const int e = oasis::check_launch("gemv_f32");
    if (e != OASIS_OK) return e;
  }
  return OASIS_OK;
}

}  // namespace oasis

extern "C" int oasis_gemv_f32(const float* x, int64_t ldx, int64_t R, const float* W, int64_t N, int64_t K,
                              const float* b, float* out, int64_t ld_out, int act_in, int act_out, int accumulate,
                              oasis_stream_t stream) {
  return oasis::gemv_f32_cat(x, ldx, K, nullptr, 0, R, W, N, K, b, out, ld_out, act_in, act_out, accumulate,
                             static_cast<hipStream_t>(stream));
}
