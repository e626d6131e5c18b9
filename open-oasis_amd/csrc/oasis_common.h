// Shared device helpers for the Oasis gfx950 kernels.
//
// Storage types: activations that feed MFMA are bf16; the residual stream,
// adaLN parameters, biases, RoPE tables and all accumulators are fp32.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <string.h>

#include "oasis_hip.h"

typedef __bf16 bf16;
typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;

#define OASIS_DEV static __device__ __forceinline__

// ---- error reporting (host) -------------------------------------------------
namespace oasis {
// Byte ranges that a kernel's extra workgroups (grid slice blockIdx.z == 1) read ahead of later
// kernels, so that their operands come from the memory-side cache instead of HBM: one 4-byte word
// per 128-byte line, the values dropped (prefetch_lines). Unused ranges have 0 bytes.
struct Prefetch {
  const void* p[4];
  int64_t bytes[4];
  int line_log2;  // bytes between the words read: 1 << line_log2 (7: one word per 128-byte line)
};
inline bool prefetch_any(const Prefetch* pf) {
  return pf && (pf->bytes[0] > 0 || pf->bytes[1] > 0 || pf->bytes[2] > 0 || pf->bytes[3] > 0);
}
inline Prefetch prefetch_or_none(const Prefetch* pf) {
  return prefetch_any(pf) ? *pf : Prefetch{{nullptr, nullptr, nullptr, nullptr}, {0, 0, 0, 0}, 7};
}
// appends a range (ignored past four)
inline void prefetch_add(Prefetch& pf, const void* p, int64_t bytes) {
  for (int i = 0; i < 4; ++i)
    if (pf.bytes[i] == 0) {
      pf.p[i] = p;
      pf.bytes[i] = bytes;
      return;
    }
}
void set_error(const char* fmt, ...);
int check_launch(const char* what);
// acc = A[M,K] @ B[N,K]^T with the given epilogue (gemm.hip).
int gemm_launch(const __bf16* A, int64_t lda, const __bf16* B, int64_t ldb, int64_t M, int64_t N, int64_t K,
                const oasis_epilogue_t& epi, hipStream_t s);
// both operands in MFMA fragment order (A with a_rows >= M rows), M <= 320 (gemm.hip)
// pf: byte ranges that workgroups past the tiles read ahead, on the CUs the tiles leave idle (up
// to 256 workgroups in all).
int gemm_frag_launch(const __bf16* A, int64_t a_rows, const __bf16* B, int64_t M, int64_t N, int64_t K,
                     const oasis_epilogue_t& epi, int splits, hipStream_t s, const Prefetch* pf = nullptr);
// rows of A any fragment-order product of M rows may read (its row tiles rounded up: 48 rows at
// most 160 tokens, 48 or 80 above)
int64_t gemm_frag_rows(int64_t M);
// explicit tile configuration and split-K count (splits > 1 needs OASIS_EPI_PARTIAL_F32). pf: byte
// ranges that workgroups past the tiles read ahead, on the CUs the wave-split tiles leave idle
// (those tiles only; up to 256 workgroups in all).
int gemm_launch_cfg(const __bf16* A, int64_t lda, const __bf16* B, int64_t ldb, int64_t M, int64_t N, int64_t K,
                    const oasis_epilogue_t& epi, int tile, int splits, hipStream_t s, const Prefetch* pf = nullptr);
// split-K count the default tile of a large-token (M >= 2048) split-K product wants
int gemm_auto_splits(int64_t M, int64_t N, int64_t K, int max_splits);
// acc = A[M,K] @ (Bq[N,K] (e4m3) * w_scale[N])^T with the given epilogue (gemm_fp8.hip).
// A_scale == nullptr: A is bf16; else A is e4m3 blocks with e8m0 scales A_scale[M, lds].
int gemm_fp8_launch(const void* A, int64_t lda, const uint8_t* A_scale, int64_t lds, const uint8_t* B, int64_t ldb,
                    const float* w_scale, int64_t M, int64_t N, int64_t K, const oasis_epilogue_t& epi, int tile,
                    int splits, hipStream_t s);
// oasis_residual_ln with an optional fp8-block LN output (y8 e4m3 [M, D], y8_scale e8m0
// [M, D/32]) in place of the bf16 one (norm.hip).
// y_frag: the bf16 output in MFMA fragment order (below 2048 rows). mean_out: each row's mean
// (after the residual), [M] fp32 (below 2048 rows, with an LN output).
int residual_ln(float* x, int64_t M, int64_t D, const float* partial, int n_partials, int64_t partial_stride,
                const float* bias, const float* gate, int64_t gate_fstride, int64_t rows_per_frame, const float* ln_a,
                const float* ln_b, int64_t ln_fstride, void* y_bf16, uint8_t* y8, uint8_t* y8_scale, float eps,
                hipStream_t s, bool y_frag = false, float* mean_out = nullptr, const Prefetch* pf = nullptr);
// The DiT's final layer in fp32 (norm.hip): the pending residual (n_partials split-K slices +
// bias, gated), LN, modulate with the frame's (scale_p1, shift) rows, then v_out[M, 64] =
// h @ W^T + b with W fp32 [64, D]. With chunk set, rows chunk_row0.. also take one DDIM step of
// chunk [M - chunk_row0, 64] with those v rows (ddim: host array of the 6 coefficients, in
// oasis_ddim_update order).
int final_layer(float* x, int64_t M, int64_t D, const float* partial, int n_partials, int64_t partial_stride,
                const float* bias, const float* gate, int64_t gate_fstride, int64_t rows_per_frame, const float* scale_p1,
                const float* shift, int64_t ada_fstride, const float* W, const float* b, float* v_out, float eps,
                hipStream_t s, float* chunk = nullptr, int64_t chunk_row0 = 0, const float* ddim = nullptr);
// oasis_gemv_f32 whose multiplied row is two inputs side by side: columns [0, K1) from x
// [R, ldx] and [K1, K) from x2 [R, ldx2] (gemv.hip).
int gemv_f32_cat(const float* x, int64_t ldx, int64_t K1, const float* x2, int64_t ldx2, int64_t R, const float* W,
                 int64_t N, int64_t K, const float* b, float* out, int64_t ld_out, int act_in, int act_out,
                 int accumulate, hipStream_t s);
// Both adaLN projections of R <= 8 rows in one launch: W16 bf16 in 16-row tile order and W32
// fp32, each applied to silu(x) (gemv.hip). Returns 1, launching nothing, for shapes it does not
// cover (the caller then runs oasis_gemv_bf16_tiled and oasis_gemv_f32).
int gemv_adaln_pair(const float* x, int64_t ldx, int64_t R, const void* W16, int64_t N16, const float* b16,
                    float* out16, const float* W32, int64_t N32, const float* b32, float* out32, int64_t K,
                    int64_t ld_out, hipStream_t s);
// Causal temporal attention (attention.hip); q_frame >= 0 computes only that query frame of
// each group and writes it as a single frame: out [B*P, n_heads*64].
// out_frag: out in MFMA fragment order (as a [rows, n_heads*64] matrix).
// pf: byte ranges read by extra workgroups beside the attention.
// out8 / out8_scale: the output as fp8 activation blocks instead of bf16 (row-major, e4m3 bytes
// [rows, n_heads*64] and e8m0 scales [rows, n_heads*2]), as oasis_quantize_act_fp8 of the bf16
// output would give; out is then not written.
int temporal_attention(const void* q, const void* k, const void* v, void* out, int64_t B, int64_t T, int64_t P,
                       int64_t n_heads, float scale, int q_frame, hipStream_t stream, bool out_frag = false,
                       const Prefetch* pf = nullptr, uint8_t* out8 = nullptr, uint8_t* out8_scale = nullptr);
// oasis_attention (heads-first q/k/v per frame, token-major out), out optionally in fragment
// order or as fp8 activation blocks (as temporal_attention), with byte ranges read by extra
// workgroups beside it.
int attention(const void* q, const void* k, const void* v, void* out, int64_t n_frames, int64_t L, int64_t n_heads,
              float scale, hipStream_t stream, bool out_frag, const Prefetch* pf, uint8_t* out8 = nullptr,
              uint8_t* out8_scale = nullptr);
// oasis_attention with out in fragment order.
int attention_frag(const void* q, const void* k, const void* v, void* out, int64_t n_frames, int64_t L,
                   int64_t n_heads, float scale, hipStream_t stream);
// QKV projection + temporal RoPE + causal attention of a two-frame temporal window in one
// kernel (temporal_qkv.hip). A: LN output [B*T*P, lda]; W: QKV weight [3D, D] (D = 64 H);
// out: attention output [B*T*P, D]. T = 2: both frames (kc / vc, optional, receive both frames'
// rotated K and V as cache slots 0 and 1); T = 1: the current frame (RoPE position 1)
// against cache slot 0. The cache is [B][P][H][2][64] bf16. P must be a multiple of 16.
int temporal_qkv_attention(const __bf16* A, int64_t lda, const __bf16* W, __bf16* out, int64_t B, int64_t T,
                           int64_t P, int64_t H, const float* t_cos, const float* t_sinp, __bf16* kc, __bf16* vc,
                           float scale, hipStream_t stream);
}  // namespace oasis

#define OASIS_REQUIRE(cond, code, ...)          \
  do {                                          \
    if (!(cond)) {                              \
      oasis::set_error(__VA_ARGS__);            \
      return (code);                            \
    }                                           \
  } while (0)

// true when every given pointer (null allowed) is a multiple of `a` bytes: the kernels move 16-,
// 8- or 4-byte vectors from their base pointers
template <typename... P>
inline bool oasis_aligned(size_t a, const P*... p) {
  const uintptr_t m = (0 | ... | reinterpret_cast<uintptr_t>(p));
  return (m & (a - 1)) == 0;
}

// Word 0 of line ll of a Prefetch's ranges taken back to back (0 past their end).
OASIS_DEV uint32_t prefetch_word(const oasis::Prefetch& pf, int64_t ll) {
  const int sh = pf.line_log2, ws = sh - 2;
  const int64_t l0 = pf.bytes[0] >> sh, l1 = l0 + (pf.bytes[1] >> sh), l2 = l1 + (pf.bytes[2] >> sh),
                l3 = l2 + (pf.bytes[3] >> sh);
  const uint32_t* p0 = static_cast<const uint32_t*>(pf.p[0]);
  const uint32_t* p1 = static_cast<const uint32_t*>(pf.p[1]);
  const uint32_t* p2 = static_cast<const uint32_t*>(pf.p[2]);
  const uint32_t* p3 = static_cast<const uint32_t*>(pf.p[3]);
  return ll < l0   ? p0[ll << ws]
         : ll < l1 ? p1[(ll - l0) << ws]
         : ll < l2 ? p2[(ll - l1) << ws]
         : ll < l3 ? p3[(ll - l2) << ws]
                   : 0u;
}

// keeps loaded words alive without using them: the loads stay and complete before this point
OASIS_DEV void prefetch_sink(uint32_t x) { __asm__ volatile("" ::"v"(x)); }


// Thread i of n reads lines i, i + n, ... of a Prefetch's ranges, U at a time, and drops the values.
template <int U>
OASIS_DEV void prefetch_part(const oasis::Prefetch& pf, int64_t i, int64_t n) {
  const int sh = pf.line_log2;
  const int64_t lines = (pf.bytes[0] >> sh) + (pf.bytes[1] >> sh) + (pf.bytes[2] >> sh) + (pf.bytes[3] >> sh);
  uint32_t acc = 0;
  for (int64_t l = i; l < lines; l += U * n) {
    uint32_t v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = prefetch_word(pf, l + u * n);
#pragma unroll
    for (int u = 0; u < U; ++u) acc ^= v[u];
  }
  prefetch_sink(acc);
}

// The prefetching workgroups' part of a Prefetch: the grid slice blockIdx.z == 1 reads one 4-byte
// word of every line of the ranges, 8 lines per thread at a time.
OASIS_DEV void prefetch_lines(const oasis::Prefetch& pf) {
  prefetch_part<8>(pf, ((int64_t)blockIdx.y * gridDim.x + blockIdx.x) * blockDim.x + threadIdx.x,
                   (int64_t)gridDim.x * gridDim.y * blockDim.x);
}

// ---- conversions ------------------------------------------------------------
OASIS_DEV float bf2f(bf16 v) { return (float)v; }
OASIS_DEV bf16 f2bf(float v) { return (bf16)v; }  // round-to-nearest-even

OASIS_DEV bf16x8 pack8(const float* v) {
  bf16x8 r;
#pragma unroll
  for (int i = 0; i < 8; ++i) r[i] = f2bf(v[i]);
  return r;
}

OASIS_DEV void unpack8(bf16x8 p, float* v) {
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = bf2f(p[i]);
}

// ---- MFMA fragment order ------------------------------------------------------
// Element (m, c) of a bf16 matrix of ks * 32 columns stored in fragment order: block (m / 16,
// c / 32) of 512 elements, piece (m % 16) + 16 ((c / 8) % 4) of 8, element c % 8. A run of 4 or 8
// columns starting at a multiple of 4 or 8 stays inside one piece.
OASIS_DEV int64_t frag_index(int64_t m, int64_t c, int64_t ks) {
  return ((((m >> 4) * ks + (c >> 5)) * 64 + (m & 15) + ((c >> 3) & 3) * 16) << 3) + (c & 7);
}

// ---- streaming accesses -----------------------------------------------------
// Non-temporal vector loads and stores (the `nt` cache policy): for data a kernel touches once.
// A streamed store leaves the L2 early instead of waiting, dirty, for the write-back at the
// kernel's end, so a memory-bound kernel's writes overlap its reads.
template <typename V>
OASIS_DEV void st_stream(V* p, V v) { __builtin_nontemporal_store(v, p); }
template <typename V>
OASIS_DEV V ld_stream(const V* p) { return __builtin_nontemporal_load(p); }

// ---- buffer loads -----------------------------------------------------------
// A scalar base (the buffer resource, made from a wave-uniform pointer) plus a 32-bit per-lane
// byte offset voff and a scalar byte offset soff: such loads move ~1.35x the bytes per cycle of
// loads with 64-bit per-lane addresses (measured from L2 with 4 waves per CU: 41 against 31 bytes
// per clock per CU).
OASIS_DEV __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base) {
  // raw buffer (stride 0), every 32-bit offset in range, 32-bit data format
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, 0xffffffff, 0x00020000);
}

// ---- cross-lane reductions without LDS --------------------------------------
// DPP moves within 16-lane rows and the gfx950 row / half-wave swaps are one VALU instruction
// each, where __shfl_xor is an LDS permute (ds_bpermute) with an LDS round trip: a 64-lane sum
// takes ~110 ns against ~260 ns in a dependent chain. Every lane pairs with a partner that pairs
// back (l ^ 1, l ^ 2, 7 - l and 15 - l within rows, l ^ 16, l ^ 32) and a + b == b + a exactly,
// so all lanes of a group end with bit-identical results. All lanes of the group must be active.
template <int CTRL>
OASIS_DEV float dpp_mov(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, true));
}
constexpr int DPP_XOR1 = 0xB1;         // quad_perm [1, 0, 3, 2]
constexpr int DPP_XOR2 = 0x4E;         // quad_perm [2, 3, 0, 1]
constexpr int DPP_HALF_MIRROR = 0x141; // lane i <-> 7 - i within each 8 lanes
constexpr int DPP_MIRROR = 0x140;      // lane i <-> 15 - i within each 16 lanes

// v_permlane16_swap (rows 0 <-> 1 and 2 <-> 3 between the two registers) and v_permlane32_swap
// (lanes 0-31 <-> 32-63), as inline asm with both registers read and written: this compiler's
// builtins return the second register's new value as the first's. Two wait states on each side.
OASIS_DEV void swap_rows16(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane16_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
OASIS_DEV void swap_halves32(float& a, float& b) {
  asm volatile("s_nop 1\n\tv_permlane32_swap_b32 %0, %1\n\ts_nop 1" : "+v"(a), "+v"(b));
}
// v op v[lane ^ 16] and v op v[lane ^ 32]: after the swap of two copies of v, a holds the even
// row's (lower half's) value and b the odd row's (upper half's) in every lane
OASIS_DEV float sum_xor16(float v) {
  float a = v, b = v;
  swap_rows16(a, b);
  return a + b;
}
OASIS_DEV float max_xor16(float v) {
  float a = v, b = v;
  swap_rows16(a, b);
  return fmaxf(a, b);
}
OASIS_DEV float sum_xor32(float v) {
  float a = v, b = v;
  swap_halves32(a, b);
  return a + b;
}
OASIS_DEV float max_xor32(float v) {
  float a = v, b = v;
  swap_halves32(a, b);
  return fmaxf(a, b);
}
// over aligned groups of 4, 8 and 16 lanes
OASIS_DEV float quad_max(float v) {
  v = fmaxf(v, dpp_mov<DPP_XOR1>(v));
  return fmaxf(v, dpp_mov<DPP_XOR2>(v));
}
// sum over the 4 lanes of a quad (every lane of the quad gets the same value)
OASIS_DEV float quad_sum(float v) {
  v += dpp_mov<DPP_XOR1>(v);
  return v + dpp_mov<DPP_XOR2>(v);
}
OASIS_DEV float oct_max(float v) {
  v = quad_max(v);
  return fmaxf(v, dpp_mov<DPP_HALF_MIRROR>(v));
}
OASIS_DEV float row16_sum(float v) {
  v += dpp_mov<DPP_XOR1>(v);
  v += dpp_mov<DPP_XOR2>(v);
  v += dpp_mov<DPP_HALF_MIRROR>(v);
  return v + dpp_mov<DPP_MIRROR>(v);
}
OASIS_DEV float row16_max(float v) {
  v = oct_max(v);
  return fmaxf(v, dpp_mov<DPP_MIRROR>(v));
}

// One DDIM step of a latent element x with predicted v (oasis_inference.py:1919-1931):
// x0 = c0 x - c1 v, eps = (c2 x - x0) c3, returns c4 x0 + c5 eps. The stand-alone update and
// the final layer's fused update share it, so both round the same way.
struct DdimCoeffs {
  float c[6];
};
OASIS_DEV float ddim_step(float x, float v, const DdimCoeffs& k) {
  const float x0 = k.c[0] * x - k.c[1] * v;
  const float eps = (k.c[2] * x - x0) * k.c[3];
  return k.c[4] * x0 + k.c[5] * eps;
}

// ---- wave reductions (64 lanes) ---------------------------------------------
OASIS_DEV float wave_sum(float v) { return sum_xor32(sum_xor16(row16_sum(v))); }
OASIS_DEV float wave_max(float v) { return max_xor32(max_xor16(row16_max(v))); }

// Sums of N values (N a power of two, 2..64) across the 64 lanes at once, v[i] holding this
// lane's part of value i. Recursive halving: at each level every lane keeps the half of its
// values selected by one lane bit and adds its partner's copy of that half (N/2 + N/4 + ... + 1
// shuffles instead of 6 per value); the lane bits left over at the end are plain sums. On return
// v[0] of lane l holds the full sum of value l / (64 / N). CNT is the level's count (template,
// so every index is a compile-time constant).
template <int N, int CNT = N>
OASIS_DEV void wave_sum_n(float* v, int lane) {
  static_assert(N >= 2 && N <= 64 && (N & (N - 1)) == 0, "N must be a power of two in [2, 64]");
  if constexpr (CNT > 1) {
    constexpr int o = 32 * CNT / N;
    const bool upper = (lane & o) != 0;
#pragma unroll
    for (int i = 0; i < CNT / 2; ++i) {
      const float give = upper ? v[i] : v[i + CNT / 2];
      const float keep = upper ? v[i + CNT / 2] : v[i];
      v[i] = keep + __shfl_xor(give, o, 64);
    }
    wave_sum_n<N, CNT / 2>(v, lane);
  } else {
#pragma unroll
    for (int o = 32 / N; o >= 1; o >>= 1) v[0] += __shfl_xor(v[0], o, 64);
  }
}

// ---- activations ------------------------------------------------------------
// tanh-GELU as x * sigmoid(2u), u = sqrt(2/pi) (x + 0.044715 x^3), i.e. x / (1 + 2^t) with
// t = -2 u log2(e), on the hardware exp2 and reciprocal (about 1 ulp each; the results are
// stored as bf16 or e4m3). Large |x| saturates to x or -0.
OASIS_DEV float gelu_tanh(float x) {
  constexpr float c1 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;
  constexpr float c3 = c1 * 0.044715f;
  const float t = x * fmaf(c3, x * x, c1);
  return x * __builtin_amdgcn_rcpf(1.0f + __builtin_amdgcn_exp2f(t));
}

// erf-GELU as the reference computes it in fp32 (torch's exact GELU): 0.5 x (1 + erf(x / sqrt 2)),
// so past x ~ -5.5 it is 0 there as here
OASIS_DEV float gelu_erf(float x) { return 0.5f * x * (1.0f + erff(x * 0.7071067811865476f)); }

OASIS_DEV float silu(float x) { return x / (1.0f + __expf(-x)); }

// ---- fp8 (OCP e4m3) activation blocks -----------------------------------------
// A block of values with max |v| = amax gets the power-of-two scale 2^(sb-127) (sb is the
// e8m0 byte) that maps amax into [128, 256): amax = m 2^(E-127), m in [1, 2) -> sb = E - 7.
OASIS_DEV int fp8_block_scale(float amax) {
  const int E = (__float_as_int(amax) >> 23) & 0xff;
  return E > 7 ? E - 7 : 0;
}
// 1 / 2^(sb-127), exact
OASIS_DEV float fp8_block_inv(int sb) { return __int_as_float((254 - sb) << 23); }
// four values -> four e4m3 bytes (round to nearest even), little-endian in a u32
OASIS_DEV uint32_t pack4_fp8(float a, float b, float c, float d) {
  int r = __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false);
  r = __builtin_amdgcn_cvt_pk_fp8_f32(c, d, r, true);
  return (uint32_t)r;
}

// ---- XCD-aware workgroup order --------------------------------------------
// MI355X dispatches workgroup i of a launch to XCD i % 8 (each XCD has its own L2). xcd_remap
// maps the dispatch id to a work id such that every XCD receives a contiguous range of work ids,
// so work items that share operands (the M tiles of one weight block, the query blocks of one
// attention head) are fetched into one L2. A bijection on [0, G): it decides locality only.
constexpr int NUM_XCD = 8;
OASIS_DEV int xcd_remap(int pid, int G) {
  const int q = G / NUM_XCD, r = G % NUM_XCD;
  const int xcd = pid % NUM_XCD, local = pid / NUM_XCD;
  return xcd < r ? xcd * (q + 1) + local : r * (q + 1) + (xcd - r) * q + local;
}

// ---- MFMA -------------------------------------------------------------------
// v_mfma_f32_16x16x32_bf16: lane l supplies A[l%16][8*(l/16)+j] and
// B[8*(l/16)+j][l%16] (j=0..7) and receives D[4*(l/16)+i][l%16] (i=0..3).
OASIS_DEV f32x4 mfma16(bf16x8 a, bf16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
