// Single-pass LayerNorm kernels: one 64-lane wave per row, the row held in registers
// (D/64 floats per lane, 16 B vector loads), mean and variance by two wave reductions
// over the registers (exact two-pass arithmetic, one HBM read), then the modulation or
// affine transform fused into the store.
//
//   ln_modulate:  y_bf16 = LN(x) * scale_p1[frame] + shift[frame]   (DiT, no affine)
//   ln_affine:    y_bf16 = LN(x) * w + b                            (VAE)
//   layernorm:    reference surface, fp32/bf16 in and out, w/b optionally row-expanded
#include "oasis_common.h"

namespace {

template <typename T>
__device__ __forceinline__ void load4(const T* p, float* v);
template <>
__device__ __forceinline__ void load4<float>(const float* p, float* v) {
  const f32x4 t = *reinterpret_cast<const f32x4*>(p);
  v[0] = t[0]; v[1] = t[1]; v[2] = t[2]; v[3] = t[3];
}
template <>
__device__ __forceinline__ void load4<bf16>(const bf16* p, float* v) {
  const bf16x4 t = *reinterpret_cast<const bf16x4*>(p);
  v[0] = bf2f(t[0]); v[1] = bf2f(t[1]); v[2] = bf2f(t[2]); v[3] = bf2f(t[3]);
}

template <typename T>
__device__ __forceinline__ void store4(T* p, const float* v);
template <>
__device__ __forceinline__ void store4<float>(float* p, const float* v) {
  *reinterpret_cast<f32x4*>(p) = f32x4{v[0], v[1], v[2], v[3]};
}
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, const float* v) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{f2bf(v[0]), f2bf(v[1]), f2bf(v[2]), f2bf(v[3])};
}

// mode 0: modulate with per-frame (shift, scale_p1); mode 1: affine (w, b) with row stride.
template <int NC, typename TIn, typename TOut, int MODE>
__global__ __launch_bounds__(256) void ln_kernel(const TIn* __restrict__ x, int64_t M, float eps,
                                                 const float* __restrict__ p0, const float* __restrict__ p1,
                                                 int64_t pstride, int64_t rows_per_frame,
                                                 TOut* __restrict__ y) {
  constexpr int D = NC * 256;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const TIn* xr = x + row * D;
  float v[NC][4];
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    load4<TIn>(xr + c * 256 + lane * 4, v[c]);
    s += (v[c][0] + v[c][1]) + (v[c][2] + v[c][3]);
  }
  const float mean = wave_sum(s) * (1.0f / D);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[c][j] -= mean;
      q += v[c][j] * v[c][j];
    }
  const float rstd = rsqrtf(wave_sum(q) * (1.0f / D) + eps);
  const float* a;
  const float* b;
  if (MODE == 0) {
    const int64_t f = row / rows_per_frame;
    a = p1 + f * pstride;  // scale_p1
    b = p0 + f * pstride;  // shift
  } else {
    a = p0 + row * pstride;  // w
    b = p1 + row * pstride;  // b
  }
  TOut* yr = y + row * D;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k = c * 256 + lane * 4;
    const f32x4 av = *reinterpret_cast<const f32x4*>(a + k);
    const f32x4 bv = *reinterpret_cast<const f32x4*>(b + k);
    float o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = v[c][j] * rstd * av[j] + bv[j];
    store4<TOut>(yr + k, o);
  }
}

// The same LayerNorm with 16-byte accesses for D % 512 == 0: lane l holds columns
// v*512 + 8l .. v*512 + 8l + 7 of each 512-wide chunk v (one 16-byte bf16 vector, or two fp32).
// Rows are read and written with streaming accesses (this kernel serves the reference-surface
// LayerNorm and the VAE's first LN; the step's residual + LN kernels below keep plain stores,
// whose output the next GEMM reads: measured no faster streamed).
template <typename T>
__device__ __forceinline__ void load8(const T* p, float* v);
template <>
__device__ __forceinline__ void load8<float>(const float* p, float* v) {
  load4<float>(p, v);
  load4<float>(p + 4, v + 4);
}
template <>
__device__ __forceinline__ void load8<bf16>(const bf16* p, float* v) {
  unpack8(ld_stream(reinterpret_cast<const bf16x8*>(p)), v);
}
template <typename T>
__device__ __forceinline__ void store8(T* p, const float* v);
template <>
__device__ __forceinline__ void store8<float>(float* p, const float* v) {
  st_stream(reinterpret_cast<f32x4*>(p), f32x4{v[0], v[1], v[2], v[3]});
  st_stream(reinterpret_cast<f32x4*>(p + 4), f32x4{v[4], v[5], v[6], v[7]});
}
template <>
__device__ __forceinline__ void store8<bf16>(bf16* p, const float* v) {
  st_stream(reinterpret_cast<bf16x8*>(p), pack8(v));
}

template <int NV, typename TIn, typename TOut, int MODE>
__global__ __launch_bounds__(256) void ln8_kernel(const TIn* __restrict__ x, int64_t M, float eps,
                                                  const float* __restrict__ p0, const float* __restrict__ p1,
                                                  int64_t pstride, int64_t rows_per_frame, TOut* __restrict__ y) {
  constexpr int D = NV * 512;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const float* a;
  const float* b;
  if (MODE == 0) {
    const int64_t f = row / rows_per_frame;
    a = p1 + f * pstride;
    b = p0 + f * pstride;
  } else {
    a = p0 + row * pstride;
    b = p1 + row * pstride;
  }
  float v[NV][8], av[NV][8], bv[NV][8];
#pragma unroll
  for (int c = 0; c < NV; ++c) load8<TIn>(x + row * D + c * 512 + lane * 8, v[c]);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NV; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) s += v[c][j];
  const float mean = wave_sum(s) * (1.0f / D);
  // the affine rows (4x the row's bytes, mostly L2 hits) are fetched once the row is in: issued
  // with the row, they queue ahead of the other waves' row loads and delay the HBM reads
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    const int k = c * 512 + lane * 8;
    load8<float>(a + k, av[c]);
    load8<float>(b + k, bv[c]);
  }
  __builtin_amdgcn_sched_barrier(0);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < NV; ++c)
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      v[c][j] -= mean;
      q += v[c][j] * v[c][j];
    }
  const float rstd = rsqrtf(wave_sum(q) * (1.0f / D) + eps);
#pragma unroll
  for (int c = 0; c < NV; ++c) {
    float o[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) o[j] = v[c][j] * rstd * av[c][j] + bv[c][j];
    store8<TOut>(y + row * D + c * 512 + lane * 8, o);
  }
}

// Residual update fused with the next LayerNorm, for few rows (under 2048): one 256-thread
// workgroup per row (VPT = D/256 floats per thread, so a row's latency is spread over 4 waves),
// every load issued up front so a row costs one memory round trip; mean and variance by two
// block reductions:
//   x[m] += g * (sum_s partial[s][m] + bias)          (NP > 0; g = gate[f(m)] or 1)
//   y[m]  = LN(x[m]) * a + b                           (a, b: modulate rows or affine)
// y is bf16, row-major or (yf) in MFMA fragment order, or (y8 != nullptr, D >= 1024) fp8
// activation blocks: e4m3 bytes y8[m, :] and one e8m0 scale per 32 columns in ys[m, :] (8
// consecutive threads share a block).
template <int VPT, int NP>
__global__ __launch_bounds__(256) void residual_ln_block_kernel(float* __restrict__ x, int64_t M, const float* __restrict__ part,
                                                          int64_t pstride, const float* __restrict__ bias,
                                                          const float* __restrict__ gate, int64_t gate_fs,
                                                          int64_t rpf, const float* __restrict__ la,
                                                          const float* __restrict__ lb, int64_t ln_fs,
                                                          bf16* __restrict__ y, uint8_t* __restrict__ y8,
                                                          uint8_t* __restrict__ ys, float eps, int yf,
                                                          float* __restrict__ mean_out, oasis::Prefetch pf) {
  constexpr int D = VPT * 256;
  constexpr int NC = VPT / 4 > 0 ? VPT / 4 : 1;   // 4-float groups per thread
  constexpr int W = VPT < 4 ? VPT : 4;            // floats per group
  __shared__ float red[2][4];
  if (blockIdx.z) {  // the prefetching slice
    prefetch_lines(pf);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t row = blockIdx.x;
  const int64_t f = row / rpf;
  float* xr = x + row * D;
  float v[NC][4], pv[NP > 0 ? NP : 1][NC][4], bv[NC][4], gv[NC][4], av[NC][4], cv[NC][4];
  auto ld = [&](const float* p, float* o) {
    if (W == 4) {
      load4<float>(p, o);
    } else {
#pragma unroll
      for (int j = 0; j < W; ++j) o[j] = p[j];
    }
  };
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k = c * 1024 + tid * W;  // W == 4: groups of 1024; W < 4: one group of 256*W
#pragma unroll
    for (int j = 0; j < 4; ++j) v[c][j] = 0.f;
    ld(xr + k, v[c]);
#pragma unroll
    for (int p = 0; p < NP; ++p) ld(part + p * pstride + row * D + k, pv[p][c]);
    if (NP > 0) {
      if (bias) ld(bias + k, bv[c]); else bv[c][0] = bv[c][1] = bv[c][2] = bv[c][3] = 0.f;
      if (gate) ld(gate + f * gate_fs + k, gv[c]); else gv[c][0] = gv[c][1] = gv[c][2] = gv[c][3] = 1.f;
    }
    if (y || y8) {
      ld(la + f * ln_fs + k, av[c]);
      ld(lb + f * ln_fs + k, cv[c]);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k = c * 1024 + tid * W;
    if (NP > 0) {
#pragma unroll
      for (int j = 0; j < W; ++j) {
        float acc = bv[c][j];
#pragma unroll
        for (int p = 0; p < NP; ++p) acc += pv[p][c][j];
        v[c][j] += gv[c][j] * acc;
      }
      if (W == 4) {
        store4<float>(xr + k, v[c]);
      } else {
#pragma unroll
        for (int j = 0; j < W; ++j) xr[k + j] = v[c][j];
      }
    }
#pragma unroll
    for (int j = 0; j < W; ++j) s += v[c][j];
  }
  if (!y && !y8) return;
  s = wave_sum(s);
  if (lane == 0) red[0][wave] = s;
  __syncthreads();
  const float mean = (red[0][0] + red[0][1] + red[0][2] + red[0][3]) * (1.0f / D);
  if (mean_out && tid == 0) mean_out[row] = mean;
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int j = 0; j < W; ++j) {
      v[c][j] -= mean;
      q += v[c][j] * v[c][j];
    }
  q = wave_sum(q);
  if (lane == 0) red[1][wave] = q;
  __syncthreads();
  const float rstd = rsqrtf((red[1][0] + red[1][1] + red[1][2] + red[1][3]) * (1.0f / D) + eps);
  bf16* yr = y + row * D;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k = c * 1024 + tid * W;
    float o[4];
#pragma unroll
    for (int j = 0; j < W; ++j) o[j] = v[c][j] * rstd * av[c][j] + cv[c][j];
    if (W == 4 && y8) {
      float amax = fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3])));
      amax = oct_max(amax);
      const int sb = fp8_block_scale(amax);
      const float inv = fp8_block_inv(sb);
      *reinterpret_cast<uint32_t*>(y8 + row * D + k) = pack4_fp8(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
      if ((tid & 7) == 0) ys[row * (D / 32) + k / 32] = (uint8_t)sb;
    } else if (W == 4) {
      store4<bf16>(yf ? y + frag_index(row, k, D / 32) : yr + k, o);
    } else {
#pragma unroll
      for (int j = 0; j < W; ++j) (yf ? y[frag_index(row, k + j, D / 32)] : yr[k + j]) = f2bf(o[j]);
    }
  }
}

// The same from 2048 rows up: one 64-lane wave per row (4 rows per workgroup), the row in
// registers as NC chunks of 256 columns (4 floats per lane each), every load of the row issued
// up front; mean and variance by two wave reductions, no LDS or barriers:
//   x[m] += g * (sum_s partial[s][m] + bias)          (NP > 0; g = gate[f(m)] or 1)
//   y[m]  = LN(x[m]) * a + b                           (a, b: modulate rows or affine)
// y is bf16, or (y8 != nullptr) fp8 activation blocks: e4m3 bytes y8[m, :] and one e8m0 scale
// per 32 columns in ys[m, :] (8 consecutive lanes share a block).
template <int NC, int NP>
__global__ __launch_bounds__(256) void residual_ln_kernel(float* __restrict__ x, int64_t M, const float* __restrict__ part,
                                                          int64_t pstride, const float* __restrict__ bias,
                                                          const float* __restrict__ gate, int64_t gate_fs,
                                                          int64_t rpf, const float* __restrict__ la,
                                                          const float* __restrict__ lb, int64_t ln_fs,
                                                          bf16* __restrict__ y, uint8_t* __restrict__ y8,
                                                          uint8_t* __restrict__ ys, float eps) {
  constexpr int D = NC * 256;
  const int lane = threadIdx.x & 63;
  const int64_t row = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= M) return;
  const int64_t f = row / rpf;
  float* xr = x + row * D;
  float v[NC][4], pv[NP > 0 ? NP : 1][NC][4], bv[NC][4], gv[NC][4], av[NC][4], cv[NC][4];
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k = c * 256 + lane * 4;
    load4<float>(xr + k, v[c]);
#pragma unroll
    for (int p = 0; p < NP; ++p) load4<float>(part + p * pstride + row * D + k, pv[p][c]);
    if (NP > 0) {
      if (bias) load4<float>(bias + k, bv[c]); else bv[c][0] = bv[c][1] = bv[c][2] = bv[c][3] = 0.f;
      if (gate) load4<float>(gate + f * gate_fs + k, gv[c]); else gv[c][0] = gv[c][1] = gv[c][2] = gv[c][3] = 1.f;
    }
    if (y || y8) {
      load4<float>(la + f * ln_fs + k, av[c]);
      load4<float>(lb + f * ln_fs + k, cv[c]);
    }
  }
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    if (NP > 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        float acc = bv[c][j];
#pragma unroll
        for (int p = 0; p < NP; ++p) acc += pv[p][c][j];
        v[c][j] += gv[c][j] * acc;
      }
      store4<float>(xr + c * 256 + lane * 4, v[c]);
    }
    s += (v[c][0] + v[c][1]) + (v[c][2] + v[c][3]);
  }
  if (!y && !y8) return;
  const float mean = wave_sum(s) * (1.0f / D);
  float q = 0.f;
#pragma unroll
  for (int c = 0; c < NC; ++c)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[c][j] -= mean;
      q += v[c][j] * v[c][j];
    }
  const float rstd = rsqrtf(wave_sum(q) * (1.0f / D) + eps);
#pragma unroll
  for (int c = 0; c < NC; ++c) {
    const int k = c * 256 + lane * 4;
    float o[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) o[j] = v[c][j] * rstd * av[c][j] + cv[c][j];
    if (y8) {
      float amax = fmaxf(fmaxf(fabsf(o[0]), fabsf(o[1])), fmaxf(fabsf(o[2]), fabsf(o[3])));
      amax = oct_max(amax);
      const int sb = fp8_block_scale(amax);
      const float inv = fp8_block_inv(sb);
      *reinterpret_cast<uint32_t*>(y8 + row * D + k) = pack4_fp8(o[0] * inv, o[1] * inv, o[2] * inv, o[3] * inv);
      if ((lane & 7) == 0) ys[row * (D / 32) + k / 32] = (uint8_t)sb;
    } else {
      store4<bf16>(y + row * D + k, o);
    }
  }
}

// The DiT's final layer in one launch, fp32 end to end as the reference keeps it
// (oasis_inference.py:1497-1521). A workgroup of 8 waves takes RB = 4 rows and all 64 outputs:
//   x[m] += g * (sum_s partial[s][m] + bias)                 (NP > 0: the pending FC2 residual)
//   h[m]  = LN(x[m]) * scale_p1[f(m)] + shift[f(m)]          (fp32, kept in LDS)
//   v[m, n] = sum_k h[m, k] W[n, k] + b[n]                    (W fp32 [64, D])
// Phase 1 gives waves 0-3 one row each (the row in registers, two wave reductions); that wave
// also writes the updated row back, and no other workgroup reads the row, so the read of x and
// its write-back cannot interleave across workgroups. Phase 2: wave w owns 8 outputs, read as
// whole weight rows (lane l holds columns 4l..4l+3 of each 256-wide chunk, so each load
// instruction reads 1 KB of one row); the first NU rows' loads are issued before phase 1. Each
// lane multiplies its columns against the 4 h rows, and every (output, row) dot product is
// reduced across the wave.
template <int NC, int NP>
__global__ __launch_bounds__(512) void final_layer_kernel(float* __restrict__ x, int64_t M, const float* __restrict__ part,
                                                          int64_t pstride, const float* __restrict__ bias,
                                                          const float* __restrict__ gate, int64_t gate_fs, int64_t rpf,
                                                          const float* __restrict__ scale_p1,
                                                          const float* __restrict__ shift, int64_t ada_fs,
                                                          const float* __restrict__ W, const float* __restrict__ fb,
                                                          float* __restrict__ v_out, float eps,
                                                          float* __restrict__ chunk, int64_t chunk_row0,
                                                          DdimCoeffs ddim) {
  constexpr int D = NC * 256;
  constexpr int RB = 4;     // rows per workgroup (one wave each in phase 1)
  constexpr int NW = 8;     // outputs per wave (8 waves: all 64)
  constexpr int NU = NC <= 4 ? 4 : 2;  // weight rows in registers at once
  __shared__ __attribute__((aligned(16))) float hs[RB][D];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int64_t m0 = (int64_t)blockIdx.x * RB;
  const int nbase = wave * NW;
  f32x4 w[NU][NC];
#pragma unroll
  for (int u = 0; u < NU; ++u)
#pragma unroll
    for (int c = 0; c < NC; ++c) w[u][c] = *reinterpret_cast<const f32x4*>(W + (int64_t)(nbase + u) * D + c * 256 + 4 * lane);
  // ---- phase 1: residual + LN + modulate of row m0 + wave (waves 0..RB-1)
  if (wave < RB) {
    const int rr = wave;
    const int64_t row = m0 + rr;
    if (row >= M) {
#pragma unroll
      for (int c = 0; c < NC; ++c) *reinterpret_cast<f32x4*>(&hs[rr][c * 256 + lane * 4]) = f32x4{0.f, 0.f, 0.f, 0.f};
    } else {
      const int64_t f = row / rpf;
      float* xr = x + row * D;
      float v[NC][4];
#pragma unroll
      for (int c = 0; c < NC; ++c) load4<float>(xr + c * 256 + lane * 4, v[c]);
      if (NP > 0) {
        float pv[NP > 0 ? NP : 1][NC][4], bv[NC][4], gv[NC][4];
#pragma unroll
        for (int c = 0; c < NC; ++c) {
          const int k = c * 256 + lane * 4;
#pragma unroll
          for (int p = 0; p < NP; ++p) load4<float>(part + p * pstride + row * D + k, pv[p][c]);
          if (bias) load4<float>(bias + k, bv[c]); else bv[c][0] = bv[c][1] = bv[c][2] = bv[c][3] = 0.f;
          if (gate) load4<float>(gate + f * gate_fs + k, gv[c]); else gv[c][0] = gv[c][1] = gv[c][2] = gv[c][3] = 1.f;
        }
#pragma unroll
        for (int c = 0; c < NC; ++c) {
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            float acc = bv[c][j];
#pragma unroll
            for (int p = 0; p < NP; ++p) acc += pv[p][c][j];
            v[c][j] += gv[c][j] * acc;
          }
          store4<float>(xr + c * 256 + lane * 4, v[c]);
        }
      }
      float s = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c) s += (v[c][0] + v[c][1]) + (v[c][2] + v[c][3]);
      const float mean = wave_sum(s) * (1.0f / D);
      float q = 0.f;
#pragma unroll
      for (int c = 0; c < NC; ++c)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          v[c][j] -= mean;
          q += v[c][j] * v[c][j];
        }
      const float rstd = rsqrtf(wave_sum(q) * (1.0f / D) + eps);
      const float* a = scale_p1 + f * ada_fs;
      const float* b = shift + f * ada_fs;
#pragma unroll
      for (int c = 0; c < NC; ++c) {
        const int k = c * 256 + lane * 4;
        const f32x4 av = *reinterpret_cast<const f32x4*>(a + k);
        const f32x4 bv = *reinterpret_cast<const f32x4*>(b + k);
        *reinterpret_cast<f32x4*>(&hs[rr][k]) = f32x4{v[c][0] * rstd * av[0] + bv[0], v[c][1] * rstd * av[1] + bv[1],
                                                      v[c][2] * rstd * av[2] + bv[2], v[c][3] * rstd * av[3] + bv[3]};
      }
    }
  }
  __syncthreads();
  // ---- phase 2: this lane's columns of the 4 h rows against the wave's 8 weight rows; the next
  // NU weight rows are in flight while the current ones are multiplied
  float part_sum[NW * RB];  // (output u, row r) at u * RB + r, this lane's columns only
#pragma unroll
  for (int nb = 0; nb < NW; nb += NU) {
    f32x4 wn[NU][NC];
    if (nb + NU < NW) {
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int c = 0; c < NC; ++c)
          wn[u][c] = *reinterpret_cast<const f32x4*>(W + (int64_t)(nbase + nb + NU + u) * D + c * 256 + 4 * lane);
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      f32x4 hv[NC];
#pragma unroll
      for (int c = 0; c < NC; ++c) hv[c] = *reinterpret_cast<const f32x4*>(&hs[r][c * 256 + 4 * lane]);
#pragma unroll
      for (int u = 0; u < NU; ++u) {
        float acc = 0.f;
#pragma unroll
        for (int c = 0; c < NC; ++c)
          acc = fmaf(hv[c][3], w[u][c][3], fmaf(hv[c][2], w[u][c][2], fmaf(hv[c][1], w[u][c][1],
                fmaf(hv[c][0], w[u][c][0], acc))));
        part_sum[(nb + u) * RB + r] = acc;
      }
    }
    if (nb + NU < NW) {
#pragma unroll
      for (int u = 0; u < NU; ++u)
#pragma unroll
        for (int c = 0; c < NC; ++c) w[u][c] = wn[u][c];
    }
  }
  // the 32 sums across the wave: lane l ends with (output, row) index l >> 1
  static_assert(NW * RB == 32, "one value per lane pair");
  wave_sum_n<NW * RB>(part_sum, lane);
  const float total = part_sum[0];
  const int idx = lane >> 1, u = idx / RB, r = idx % RB;
  const int64_t row = m0 + r;
  const int n = nbase + u;
  if ((lane & 1) == 0 && row < M) {
    const float vo = total + (fb ? fb[n] : 0.f);
    v_out[row * 64 + n] = vo;
    // the fused DDIM step: rows from chunk_row0 on are the denoised frame, chunk [., 64]
    if (chunk && row >= chunk_row0) {
      float* cp = chunk + (row - chunk_row0) * 64 + n;
      *cp = ddim_step(*cp, vo, ddim);
    }
  }
}

template <int NC>
hipError_t final_layer_np(int np, float* x, int64_t M, const float* part, int64_t ps, const float* bias,
                          const float* gate, int64_t gfs, int64_t rpf, const float* scale_p1, const float* shift,
                          int64_t afs, const float* W, const float* fb, float* v_out, float eps, float* chunk,
                          int64_t chunk_row0, const DdimCoeffs& dc, hipStream_t s) {
  const dim3 grid((unsigned)((M + 3) / 4)), block(512);  // 4 rows and all 64 outputs per workgroup
#define OASIS_FIN(NPV)                                                                                            \
  hipLaunchKernelGGL((final_layer_kernel<NC, NPV>), grid, block, 0, s, x, M, part, ps, bias, gate, gfs, rpf, scale_p1, \
                     shift, afs, W, fb, v_out, eps, chunk, chunk_row0, dc)
  switch (np) {
    case 0: OASIS_FIN(0); break;
    case 1: OASIS_FIN(1); break;
    case 2: OASIS_FIN(2); break;
    case 3: OASIS_FIN(3); break;
    case 4: OASIS_FIN(4); break;
    case 8: OASIS_FIN(8); break;
    default: return hipErrorInvalidConfiguration;
  }
#undef OASIS_FIN
  return hipGetLastError();
}

template <int NC>
hipError_t residual_ln_np(int np, float* x, int64_t M, const float* part, int64_t ps, const float* bias,
                          const float* gate, int64_t gfs, int64_t rpf, const float* la, const float* lb, int64_t lfs,
                          bf16* y, uint8_t* y8, uint8_t* ys, float eps, hipStream_t s, int yf, float* mean_out,
                          const oasis::Prefetch& pf) {
  // few rows: a 256-thread workgroup per row (VPT = NC floats per thread), plus the prefetching
  // slice when pf names ranges; many: a wave per row
  const bool wave_rows = M >= 2048;
  const dim3 grid((unsigned)(wave_rows ? (M + 3) / 4 : M)), block(256);
  const dim3 grid_pf((unsigned)M, 1, oasis::prefetch_any(&pf) ? 2 : 1);
#define OASIS_RLN(NPV)                                                                                          \
  if (wave_rows)                                                                                                \
    hipLaunchKernelGGL((residual_ln_kernel<NC, NPV>), grid, block, 0, s, x, M, part, ps, bias, gate, gfs, rpf, la, \
                       lb, lfs, y, y8, ys, eps);                                                                \
  else                                                                                                          \
    hipLaunchKernelGGL((residual_ln_block_kernel<NC, NPV>), grid_pf, block, 0, s, x, M, part, ps, bias, gate, gfs,  \
                       rpf, la, lb, lfs, y, y8, ys, eps, yf, mean_out, pf)
  switch (np) {
    case 0: OASIS_RLN(0); break;
    case 1: OASIS_RLN(1); break;
    case 2: OASIS_RLN(2); break;
    case 3: OASIS_RLN(3); break;
    case 4: OASIS_RLN(4); break;
    case 8: OASIS_RLN(8); break;
    default: return hipErrorInvalidConfiguration;
  }
#undef OASIS_RLN
  return hipGetLastError();
}

template <typename TIn, typename TOut, int MODE>
hipError_t ln_dispatch(const TIn* x, int64_t M, int64_t D, float eps, const float* p0,
                       const float* p1, int64_t pstride, int64_t rpf, TOut* y, hipStream_t s) {
  const dim3 grid((unsigned)((M + 3) / 4)), block(256);
  switch (D) {
    case 256: hipLaunchKernelGGL((ln_kernel<1, TIn, TOut, MODE>), grid, block, 0, s, x, M, eps, p0, p1, pstride, rpf, y); break;
    case 512: hipLaunchKernelGGL((ln8_kernel<1, TIn, TOut, MODE>), grid, block, 0, s, x, M, eps, p0, p1, pstride, rpf, y); break;
    case 1024: hipLaunchKernelGGL((ln8_kernel<2, TIn, TOut, MODE>), grid, block, 0, s, x, M, eps, p0, p1, pstride, rpf, y); break;
    case 2048: hipLaunchKernelGGL((ln8_kernel<4, TIn, TOut, MODE>), grid, block, 0, s, x, M, eps, p0, p1, pstride, rpf, y); break;
    case 4096: hipLaunchKernelGGL((ln8_kernel<8, TIn, TOut, MODE>), grid, block, 0, s, x, M, eps, p0, p1, pstride, rpf, y); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

int finish(hipError_t e, const char* what) {
  if (e == hipErrorInvalidValue) {
    oasis::set_error("%s: D must be one of 256, 512, 1024, 2048, 4096", what);
    return OASIS_ERR_SHAPE;
  }
  if (e != hipSuccess) {
    oasis::set_error("%s launch failed: %s", what, hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

}  // namespace

extern "C" int oasis_ln_modulate(const float* x, int64_t M, int64_t D, const float* shift,
                                 const float* scale_p1, int64_t ada_fstride, int64_t rows_per_frame,
                                 void* y_bf16, float eps, oasis_stream_t stream) {
  OASIS_REQUIRE(x && shift && scale_p1 && y_bf16, OASIS_ERR_NULL, "ln_modulate: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, x, shift, scale_p1, y_bf16), OASIS_ERR_ARG, "ln_modulate: pointers must be 16-byte aligned");
  OASIS_REQUIRE(M > 0 && rows_per_frame > 0, OASIS_ERR_SHAPE, "ln_modulate: bad M/rows_per_frame");
  return finish(ln_dispatch<float, bf16, 0>(x, M, D, eps, shift, scale_p1, ada_fstride, rows_per_frame,
                                            static_cast<bf16*>(y_bf16), static_cast<hipStream_t>(stream)),
                "ln_modulate");
}

extern "C" int oasis_ln_affine(const float* x, int64_t M, int64_t D, const float* w, const float* b,
                               void* y_bf16, float eps, oasis_stream_t stream) {
  OASIS_REQUIRE(x && w && b && y_bf16, OASIS_ERR_NULL, "ln_affine: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, x, w, b, y_bf16), OASIS_ERR_ARG, "ln_affine: pointers must be 16-byte aligned");
  OASIS_REQUIRE(M > 0, OASIS_ERR_SHAPE, "ln_affine: bad M");
  return finish(ln_dispatch<float, bf16, 1>(x, M, D, eps, w, b, 0, 1, static_cast<bf16*>(y_bf16),
                                            static_cast<hipStream_t>(stream)),
                "ln_affine");
}

extern "C" int oasis_layernorm(const void* x, const void* weight, const void* bias, int64_t wb_ld,
                               void* out, int64_t rows, int64_t cols, float eps, int dtype,
                               oasis_stream_t stream) {
  OASIS_REQUIRE(x && weight && bias && out, OASIS_ERR_NULL, "layernorm: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, x, weight, bias, out), OASIS_ERR_ARG, "layernorm: pointers must be 16-byte aligned");
  OASIS_REQUIRE(rows > 0 && wb_ld >= 0, OASIS_ERR_SHAPE, "layernorm: bad rows/wb_ld");
  hipStream_t s = static_cast<hipStream_t>(stream);
  // weight/bias are fp32 for both dtypes (the Python surface upcasts them once).
  if (dtype == OASIS_F32)
    return finish(ln_dispatch<float, float, 1>(static_cast<const float*>(x), rows, cols, eps,
                                               static_cast<const float*>(weight), static_cast<const float*>(bias),
                                               wb_ld, 1, static_cast<float*>(out), s),
                  "layernorm");
  if (dtype == OASIS_BF16)
    return finish(ln_dispatch<bf16, bf16, 1>(static_cast<const bf16*>(x), rows, cols, eps,
                                             static_cast<const float*>(weight), static_cast<const float*>(bias),
                                             wb_ld, 1, static_cast<bf16*>(out), s),
                  "layernorm");
  oasis::set_error("layernorm: unsupported dtype %d", dtype);
  return OASIS_ERR_DTYPE;
}

namespace oasis {

int residual_ln(float* x, int64_t M, int64_t D, const float* partial, int n_partials, int64_t partial_stride,
                const float* bias, const float* gate, int64_t gate_fstride, int64_t rows_per_frame, const float* ln_a,
                const float* ln_b, int64_t ln_fstride, void* y_bf16, uint8_t* y8, uint8_t* y8_scale, float eps,
                hipStream_t s, bool y_frag, float* mean_out, const Prefetch* pf) {
  OASIS_REQUIRE(x, OASIS_ERR_NULL, "residual_ln: null x");
  const Prefetch pfv = prefetch_or_none(M < 2048 ? pf : nullptr);
  OASIS_REQUIRE(!mean_out || (M < 2048 && (y_bf16 || y8)), OASIS_ERR_ARG,
                "residual_ln: row means are written for M < 2048 with an LN output");
  OASIS_REQUIRE(!y_frag || (M < 2048 && M % 16 == 0 && !y8), OASIS_ERR_ARG,
                "residual_ln: a fragment-order output needs M < 2048, M %% 16 == 0 and a bf16 output");
  OASIS_REQUIRE(oasis_aligned(16, x, partial, bias, gate, ln_a, ln_b, y_bf16, y8), OASIS_ERR_ARG,
                "residual_ln: pointers must be 16-byte aligned");
  OASIS_REQUIRE(M > 0 && M < (1ll << 31) && rows_per_frame > 0, OASIS_ERR_SHAPE, "residual_ln: bad M/rows_per_frame");
  OASIS_REQUIRE(n_partials == 0 || partial, OASIS_ERR_NULL, "residual_ln: null partials");
  OASIS_REQUIRE(n_partials <= 1 || partial_stride >= M * D, OASIS_ERR_ARG, "residual_ln: partial_stride too small");
  OASIS_REQUIRE(!(y_bf16 || y8) || (ln_a && ln_b), OASIS_ERR_NULL, "residual_ln: LN output needs ln_a and ln_b");
  OASIS_REQUIRE(!y8 || (y8_scale && D >= 1024), OASIS_ERR_ARG, "residual_ln: fp8 output needs scales and D >= 1024");
  bf16* y = static_cast<bf16*>(y_bf16);
  hipError_t e;
  switch (D) {
    case 256: e = residual_ln_np<1>(n_partials, x, M, partial, partial_stride, bias, gate, gate_fstride, rows_per_frame, ln_a, ln_b, ln_fstride, y, y8, y8_scale, eps, s, y_frag ? 1 : 0, mean_out, pfv); break;
    case 512: e = residual_ln_np<2>(n_partials, x, M, partial, partial_stride, bias, gate, gate_fstride, rows_per_frame, ln_a, ln_b, ln_fstride, y, y8, y8_scale, eps, s, y_frag ? 1 : 0, mean_out, pfv); break;
    case 1024: e = residual_ln_np<4>(n_partials, x, M, partial, partial_stride, bias, gate, gate_fstride, rows_per_frame, ln_a, ln_b, ln_fstride, y, y8, y8_scale, eps, s, y_frag ? 1 : 0, mean_out, pfv); break;
    case 2048: e = residual_ln_np<8>(n_partials, x, M, partial, partial_stride, bias, gate, gate_fstride, rows_per_frame, ln_a, ln_b, ln_fstride, y, y8, y8_scale, eps, s, y_frag ? 1 : 0, mean_out, pfv); break;
    default:
      set_error("residual_ln: D=%lld must be one of 256, 512, 1024, 2048", (long long)D);
      return OASIS_ERR_SHAPE;
  }
  if (e == hipErrorInvalidConfiguration) {
    set_error("residual_ln: n_partials=%d must be one of 0-4 or 8", n_partials);
    return OASIS_ERR_ARG;
  }
  if (e != hipSuccess) {
    set_error("residual_ln launch failed: %s", hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

int final_layer(float* x, int64_t M, int64_t D, const float* partial, int n_partials, int64_t partial_stride,
                const float* bias, const float* gate, int64_t gate_fstride, int64_t rows_per_frame, const float* scale_p1,
                const float* shift, int64_t ada_fstride, const float* W, const float* b, float* v_out, float eps,
                hipStream_t s, float* chunk, int64_t chunk_row0, const float* ddim) {
  OASIS_REQUIRE(x && scale_p1 && shift && W && v_out, OASIS_ERR_NULL, "final_layer: null pointer");
  OASIS_REQUIRE(!chunk || (ddim && chunk_row0 >= 0 && chunk_row0 < M), OASIS_ERR_ARG,
                "final_layer: the fused DDIM update needs its coefficients and a first row in [0, M)");
  DdimCoeffs dc = {};
  if (chunk) memcpy(dc.c, ddim, sizeof(dc.c));
  OASIS_REQUIRE(oasis_aligned(16, x, partial, bias, gate, scale_p1, shift, W), OASIS_ERR_ARG,
                "final_layer: pointers must be 16-byte aligned");
  OASIS_REQUIRE(M > 0 && M < (1ll << 31) && rows_per_frame > 0, OASIS_ERR_SHAPE, "final_layer: bad M/rows_per_frame");
  OASIS_REQUIRE(n_partials == 0 || partial, OASIS_ERR_NULL, "final_layer: null partials");
  OASIS_REQUIRE(n_partials <= 1 || partial_stride >= M * D, OASIS_ERR_ARG, "final_layer: partial_stride too small");
  hipError_t e;
  switch (D) {
    case 256: e = final_layer_np<1>(n_partials, x, M, partial, partial_stride, bias, gate, gate_fstride, rows_per_frame, scale_p1, shift, ada_fstride, W, b, v_out, eps, chunk, chunk_row0, dc, s); break;
    case 512: e = final_layer_np<2>(n_partials, x, M, partial, partial_stride, bias, gate, gate_fstride, rows_per_frame, scale_p1, shift, ada_fstride, W, b, v_out, eps, chunk, chunk_row0, dc, s); break;
    case 1024: e = final_layer_np<4>(n_partials, x, M, partial, partial_stride, bias, gate, gate_fstride, rows_per_frame, scale_p1, shift, ada_fstride, W, b, v_out, eps, chunk, chunk_row0, dc, s); break;
    case 2048: e = final_layer_np<8>(n_partials, x, M, partial, partial_stride, bias, gate, gate_fstride, rows_per_frame, scale_p1, shift, ada_fstride, W, b, v_out, eps, chunk, chunk_row0, dc, s); break;
    default:
      set_error("final_layer: D=%lld must be one of 256, 512, 1024, 2048", (long long)D);
      return OASIS_ERR_SHAPE;
  }
  if (e == hipErrorInvalidConfiguration) {
    set_error("final_layer: n_partials=%d must be one of 0-4 or 8", n_partials);
    return OASIS_ERR_ARG;
  }
  if (e != hipSuccess) {
    set_error("final_layer launch failed: %s", hipGetErrorString(e));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

}  // namespace oasis

extern "C" int oasis_residual_ln(float* x, int64_t M, int64_t D, const float* partial, int n_partials,
                                 int64_t partial_stride, const float* bias, const float* gate, int64_t gate_fstride,
                                 int64_t rows_per_frame, const float* ln_a, const float* ln_b, int64_t ln_fstride,
                                 void* y_bf16, float eps, oasis_stream_t stream) {
  return oasis::residual_ln(x, M, D, partial, n_partials, partial_stride, bias, gate, gate_fstride, rows_per_frame,
                            ln_a, ln_b, ln_fstride, y_bf16, nullptr, nullptr, eps, static_cast<hipStream_t>(stream));
}
