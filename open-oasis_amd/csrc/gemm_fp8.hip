// fp8 weight GEMM for gfx950: bf16 activations x OCP e4m3 weights on the block-scaled
// MFMA v_mfma_scale_f32_16x16x128_f8f6f4, with the same fused epilogues as the bf16 GEMM.
//
//   acc[m, n] = sum_k A[m, k] * Wq[n, k] * w_scale[n]
//
// Weights: Wq = round_e4m3(W / w_scale[n]), w_scale[n] = max_k |W[n, k]| / 448, one fp32
// scale per output channel, stored [N, K] bytes (oasis_quantize_fp8_rows makes them).
// Activations are fp8 blocks: every 32-wide K block of a row has a power-of-two (e8m0)
// scale 2^e with the block's max |a| / 2^e in [128, 256), applied by the MFMA in hardware.
// Two A forms: bf16 in HBM, quantized by each workgroup on the way into LDS (AQ = false,
// oasis_gemm_fp8), or already quantized by the producer kernel (AQ = true,
// oasis_gemm_fp8_a8: e4m3 bytes + one scale byte per block, half the A bytes and no
// quantization work per N tile). The per-channel weight scale multiplies the fp32
// accumulator before the epilogue.
//
// MFMA operand layout (16x16x128, verified on MI355X against a host reference): lane l
// supplies row l%16 of A (column l%16 of B) with the 32 bytes k = 16g..16g+15 and
// 64+16g..64+16g+15, g = l/16; its scale byte covers row l%16 and K block [32g, 32g+32).
// Accumulator element r of lane l is D[4*(l/16) + r][l%16].
#include "gemm_epilogue.h"

namespace {

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float v4f __attribute__((ext_vector_type(4)));

constexpr int BK8 = 128;          // K per MFMA step and per pipeline step
constexpr int P8 = BK8;           // LDS row pitch in bytes: unpadded, 16-byte chunks XOR-swizzled

// byte offset of (row r, byte column c) in a swizzled LDS tile: 16-byte chunk c/16 of row r
// is stored at slot (c/16) ^ ((r >> 1) & 7), which keeps 16-row fragment reads conflict-free
__device__ __forceinline__ int swz(int r, int c) { return r * P8 + ((((c >> 4) ^ (r >> 1)) & 7) << 4) + (c & 15); }
constexpr int kScaleOne = 127;    // e8m0 encoding of 1.0

// Quantizes 8 consecutive bf16 of one row whose 32-wide K block is shared with the
// threads tid^1, tid^2 (same wave): returns the 8 e4m3 bytes and the block's e8m0 scale.
__device__ __forceinline__ uint2 quant8(i32x4 raw, int* sbyte) {
  const bf16x8 h = __builtin_bit_cast(bf16x8, raw);
  float v[8];
  float amax = 0.f;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    v[j] = (float)h[j];
    amax = fmaxf(amax, fabsf(v[j]));
  }
  amax = quad_max(amax);
  const int sb = fp8_block_scale(amax);
  const float inv = fp8_block_inv(sb);
  *sbyte = sb;
  return make_uint2(pack4_fp8(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv),
                    pack4_fp8(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv));
}

// v = c * s + b (weight channel scale, then bias) with the product rounded before the sum (no
// fused multiply-add), the same in every fp8 kernel, so all fp8 tiles give bit-identical outputs.
__device__ __forceinline__ void scale_bias8(f32x4 c0, f32x4 c1, f32x4 s0, f32x4 s1, f32x4 b0, f32x4 b1, float* v) {
#pragma clang fp contract(off)
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    v[j] = c0[j] * s0[j] + b0[j];
    v[j + 4] = c1[j] * s1[j] + b1[j];
  }
}

template <int BM, int BN, int WM, int WN, int STAGES, bool AQ>
__global__ __launch_bounds__(256) void gemm_fp8_kernel(const void* __restrict__ Av, int64_t lda,
                                                       const uint8_t* __restrict__ Ascale, int64_t lds,
                                                       const uint8_t* __restrict__ B, int64_t ldb,
                                                       const float* __restrict__ wscale, int M, int N, int K,
                                                       int splits, Epi e) {
  static_assert(WM * WN == 4, "4 waves");
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  static_assert(FM * 16 == TM && FN * 16 == TN, "wave tile must be a multiple of 16");
  constexpr int A_EPC = AQ ? 16 : 8;         // A elements per 16-byte chunk (fp8 or bf16)
  constexpr int A_CHUNKS = BM * (BK8 / A_EPC);
  constexpr int B_CHUNKS = BN * (BK8 / 16);  // 16-byte chunks of 16 fp8
  static_assert(A_CHUNKS % 256 == 0 && B_CHUNKS % 256 == 0, "BM multiple of 16 (32 for fp8 A), BN of 32");
  static_assert(!AQ || BM <= 256, "one scale word per thread");
  constexpr int A_PER = A_CHUNKS / 256;
  constexpr int B_PER = B_CHUNKS / 256;
  constexpr int A_BYTES = BM * P8, B_BYTES = BN * P8, S_BYTES = BM * 4;
  constexpr int RING = 2 * (A_BYTES + B_BYTES + S_BYTES);
  constexpr int C_PITCH = BN + 4;
  constexpr int C_BYTES = BM * C_PITCH * 4;
  constexpr int SMEM = RING > C_BYTES ? RING : C_BYTES;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  uint8_t* As = reinterpret_cast<uint8_t*>(smem);   // [2][BM][P8] swizzled
  uint8_t* Bs = As + 2 * A_BYTES;                   // [2][BN][P8] swizzled
  uint8_t* Ss = Bs + 2 * B_BYTES;                   // [2][BM][4] e8m0 scales of A

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  const int pid = xcd_remap(blockIdx.x, Mt * Nt * splits);
  const int mt = pid % Mt;
  const int rest = pid / Mt;
  const int split = rest % splits, nt = rest / splits;
  const int m0 = mt * BM, n0 = nt * BN;
  const int nk = K / BK8 / splits;  // the host guarantees nk % STAGES == 0
  const int kb = split * nk * BK8;

  const char* a_src[A_PER];
  int a_dst[A_PER], s_dst[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int c = tid + i * 256;
    const int row = c / (BK8 / A_EPC), col = (c % (BK8 / A_EPC)) * A_EPC;
    a_src[i] = static_cast<const char*>(Av) + ((int64_t)min(m0 + row, M - 1) * lda + kb + col) * (AQ ? 1 : 2);
    a_dst[i] = swz(row, col);
    s_dst[i] = (col & 31) == 0 ? row * 4 + col / 32 : -1;
  }
  // AQ: thread t < BM copies row t's 4 block scales of each K tile (one 32-bit word)
  const uint8_t* sc_src = AQ ? Ascale + (int64_t)min(m0 + (tid % BM), M - 1) * lds + kb / 32 : nullptr;
  const uint8_t* b_src[B_PER];
  int b_dst[B_PER];
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int c = tid + i * 256;
    const int row = c / (BK8 / 16), col = (c % (BK8 / 16)) * 16;
    b_src[i] = B + (int64_t)min(n0 + row, N - 1) * ldb + kb + col;
    b_dst[i] = swz(row, col);
  }

  i32x4 ra[STAGES][A_PER], rb[STAGES][B_PER];
  uint32_t rs[STAGES];
  auto gload = [&](int slot, int kt) {
    const int64_t ka = (int64_t)kt * BK8;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) ra[slot][i] = *reinterpret_cast<const i32x4*>(a_src[i] + ka * (AQ ? 1 : 2));
#pragma unroll
    for (int i = 0; i < B_PER; ++i) rb[slot][i] = *reinterpret_cast<const i32x4*>(b_src[i] + ka);
    if (AQ) rs[slot] = *reinterpret_cast<const uint32_t*>(sc_src + ka / 32);
  };
  auto lstore = [&](int slot, int buf) {
    uint8_t* as = As + buf * A_BYTES;
    uint8_t* bs = Bs + buf * B_BYTES;
    uint8_t* ss = Ss + buf * S_BYTES;
    if (AQ) {
#pragma unroll
      for (int i = 0; i < A_PER; ++i) *reinterpret_cast<i32x4*>(as + a_dst[i]) = ra[slot][i];
      if (tid < BM) *reinterpret_cast<uint32_t*>(ss + tid * 4) = rs[slot];
    } else {
#pragma unroll
      for (int i = 0; i < A_PER; ++i) {
        int sb;
        *reinterpret_cast<uint2*>(as + a_dst[i]) = quant8(ra[slot][i], &sb);
        if (s_dst[i] >= 0) ss[s_dst[i]] = (uint8_t)sb;
      }
    }
#pragma unroll
    for (int i = 0; i < B_PER; ++i) *reinterpret_cast<i32x4*>(bs + b_dst[i]) = rb[slot][i];
  };

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, g = lane >> 4;
  auto compute = [&](int buf) {
    const uint8_t* as = As + buf * A_BYTES;
    const uint8_t* bs = Bs + buf * B_BYTES;
    const uint8_t* ss = Ss + buf * S_BYTES + (wm * TM + lr) * 4 + g;
    i32x8 af[FM], bfr[FN];
    int sa[FM];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      const int r = wm * TM + i * 16 + lr;
      const i32x4 x0 = *reinterpret_cast<const i32x4*>(as + swz(r, 16 * g));
      const i32x4 x1 = *reinterpret_cast<const i32x4*>(as + swz(r, 64 + 16 * g));
      af[i] = i32x8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
      sa[i] = ss[i * 16 * 4];
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int r = wn * TN + j * 16 + lr;
      const i32x4 x0 = *reinterpret_cast<const i32x4*>(bs + swz(r, 16 * g));
      const i32x4 x1 = *reinterpret_cast<const i32x4*>(bs + swz(r, 64 + 16 * g));
      bfr[j] = i32x8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
    }
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(af[i], bfr[j], acc[i][j], 0, 0, 0, sa[i], 0,
                                                                      kScaleOne);
  };

#pragma unroll
  for (int s = 0; s < STAGES; ++s) gload(s, min(s, nk - 1));
  lstore(0, 0);
  __syncthreads();
  for (int k0 = 0; k0 < nk; k0 += STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s) {
      const int k = k0 + s;
      gload(s, min(k + STAGES, nk - 1));
      compute(k & 1);
      lstore((s + 1) % STAGES, (k + 1) & 1);
      __syncthreads();
    }
  }

  float* Cs = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        Cs[(wm * TM + i * 16 + g * 4 + r) * C_PITCH + wn * TN + j * 16 + lr] = acc[i][j][r];
  __syncthreads();

  constexpr int UNITS = BM * (BN / 8);
  for (int u = tid; u < UNITS; u += 256) {
    const int r = u / (BN / 8), c8 = (u % (BN / 8)) * 8;
    const int gm = m0 + r, gn = n0 + c8;
    if (gm >= M || gn >= N) continue;
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(Cs + r * C_PITCH + c8);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(Cs + r * C_PITCH + c8 + 4);
    const f32x4 s0 = *reinterpret_cast<const f32x4*>(wscale + gn);
    const f32x4 s1 = *reinterpret_cast<const f32x4*>(wscale + gn + 4);
    f32x4 b0 = f32x4{0.f, 0.f, 0.f, 0.f}, b1 = b0;
    if (e.bias && e.kind != OASIS_EPI_PARTIAL_F32) {
      b0 = *reinterpret_cast<const f32x4*>(e.bias + gn);
      b1 = *reinterpret_cast<const f32x4*>(e.bias + gn + 4);
    }
    float v[8];
    scale_bias8(c0, c1, s0, s1, b0, b1, v);
    if (e.kind == OASIS_EPI_PARTIAL_F32) {
      float* d = e.out_f32 + (int64_t)split * e.split_stride + (int64_t)gm * e.ld_out + gn;
      *reinterpret_cast<f32x4*>(d) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(d + 4) = f32x4{v[4], v[5], v[6], v[7]};
    } else {
      epilogue8(e, gm, gn, v, nullptr, 0, false);
    }
  }
}

// Large-token fp8 variant (2048+ tokens, A already in e4m3 blocks): 6 or 8 waves share a tall
// tile (288 x 256, 144 x 128 and the like, as the bf16 gemm_big_kernel) and the K tiles reach LDS
// through global_load_lds, 128 fp8 per row (one 16x16x128 MFMA step) in the same swizzled 128-byte
// rows, plus each A row's 4 block-scale bytes per K tile (4 bytes per lane, the first waves' lanes
// one row each). STAGES K tiles in the ring (two for the 288-row tiles, which is what 160 KB holds);
// the epilogue stages 16 rows of a wave's tile at a time in that wave's LDS.
template <int BM, int BN, int WM, int WN, int KIND = -1, int STAGES = 2>
__global__ __launch_bounds__(WM * WN * 64) void gemm_fp8_big_kernel(const uint8_t* __restrict__ A, int64_t lda,
                                                                   const uint8_t* __restrict__ Ascale, int64_t lds,
                                                                   const uint8_t* __restrict__ B, int64_t ldb,
                                                                   const float* __restrict__ wscale, int M, int N,
                                                                   int K, int splits, Epi e) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  static_assert(FM * 16 == TM && FN * 16 == TN, "wave tile must be a multiple of 16");
  constexpr int NBLK = (BM + BN) / 8;  // 1 KB blocks of 8 rows per stage
  static_assert(BM % 8 == 0 && BN % 8 == 0, "whole 8-row blocks");
  constexpr int LPW = (NBLK + NW - 1) / NW;
  constexpr int SWAVES = (BM + 63) / 64;  // waves that load the A scales (64 rows each)
  static_assert(SWAVES <= NW, "scale rows");
  static_assert(STAGES >= 2 && (STAGES - 2) * (LPW + 1) <= 63, "vmcnt range");
  constexpr int DATA = (BM + BN) * P8;
  // every wave issues LPW + 1 loads per stage (a wave past the scale rows reloads a clamped scale
  // word into a slot of its own), so one vmcnt bound holds for all waves
  constexpr int STAGE = DATA + NW * 256;
  constexpr int RING = STAGES * STAGE;
  constexpr int EP = TN + 4;
  constexpr int EPI_BYTES = NW * 16 * EP * 4;
  constexpr int SMEM = RING > EPI_BYTES ? RING : EPI_BYTES;
  static_assert(SMEM <= 160 * 1024, "LDS");
  constexpr int GN = 8;
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  // the wave index read back as a scalar, so that the load bases built from it stay in SGPRs
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  int split, mt, nt;
  grouped_tile(xcd_remap(blockIdx.x, Mt * Nt * splits), Mt, Nt, GN, split, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int nk = K / BK8 / splits;
  const int kb = split * nk * BK8;

  // buffer loads: the tile's first A row / weight row as the scalar base, the K tile as a scalar
  // offset, a 32-bit lane offset below BM (BN) rows of lda (ldb) bytes
  const __amdgpu_buffer_rsrc_t Ars = buffer_rsrc(A + (int64_t)m0 * lda + kb);
  const __amdgpu_buffer_rsrc_t Brs = buffer_rsrc(B + (int64_t)n0 * ldb + kb);
  uint32_t off[LPW];
  int dst[LPW];
  bool from_a[LPW];
#pragma unroll
  for (int u = 0; u < LPW; ++u) {
    const int blk = min(wave * LPW + u, NBLK - 1);
    const int r = blk * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    from_a[u] = blk * 8 < BM;  // wave-uniform: BM is a multiple of 8
    off[u] = from_a[u] ? (uint32_t)((int64_t)(min(m0 + r, M - 1) - m0) * lda + c * 16)
                       : (uint32_t)((int64_t)(min(n0 + r - BM, N - 1) - n0) * ldb + c * 16);
    dst[u] = blk * 1024;
  }
  // scale word of A row wave*64 + lane (rows past the tile load a clamped row, never read)
  const uint8_t* ssrc = Ascale + (int64_t)min(m0 + wave * 64 + lane, M - 1) * lds + kb / 32;
  auto issue = [&](int kt, int buf) {
    char* base = smem + buf * STAGE;
#pragma unroll
    for (int u = 0; u < LPW; ++u) buffer_load_lds16(from_a[u] ? Ars : Brs, off[u], kt * BK8, base + dst[u]);
    load_lds4(ssrc + kt * (BK8 / 32), base + DATA + wave * 256);
  };

  v4f acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = v4f{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, g = lane >> 4;
  auto frag = [&](const char* base, int r) -> i32x8 {
    const i32x4 x0 = *reinterpret_cast<const i32x4*>(base + r * P8 + (((g ^ (r >> 1)) & 7) << 4));
    const i32x4 x1 = *reinterpret_cast<const i32x4*>(base + r * P8 + ((((4 + g) ^ (r >> 1)) & 7) << 4));
    return i32x8{x0[0], x0[1], x0[2], x0[3], x1[0], x1[1], x1[2], x1[3]};
  };
  // B fragments first; then A fragment i + 1 and its scale byte are read while the MFMAs of
  // fragment i issue (a wait and scheduling barriers keep that order), so only two A fragments
  // are live beside the 4 * FM * FN accumulator registers and each read lands under FN MFMAs
  auto compute = [&](int buf) {
    const char* base = smem + buf * STAGE;
    const uint8_t* sb = reinterpret_cast<const uint8_t*>(base + DATA);
    i32x8 bfr[FN];
#pragma unroll
    for (int j = 0; j < FN; ++j) bfr[j] = frag(base, BM + wn * TN + j * 16 + lr);
    i32x8 a = frag(base, wm * TM + lr);
    int sa = sb[(wm * TM + lr) * 4 + g];
#pragma unroll
    for (int i = 0; i < FM; ++i) {
      // fragment i (and, at i = 0, the B fragments) landed before fragment i + 1's reads are issued,
      // so the wait never covers the reads that the MFMAs below are meant to hide
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
      i32x8 an = a;
      int sn = sa;
      if (i + 1 < FM) {
        const int rn = wm * TM + (i + 1) * 16 + lr;
        an = frag(base, rn);
        sn = sb[rn * 4 + g];
      }
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, bfr[j], acc[i][j], 0, 0, 0, sa, 0, kScaleOne);
      __builtin_amdgcn_sched_barrier(0);
      a = an;
      sa = sn;
    }
  };

  constexpr int VM = (STAGES - 2) * (LPW + 1);  // stages that may stay in flight: tile k is in LDS
  constexpr int WAIT = (VM & 15) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8);
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue(min(s, nk - 1), s);
  for (int k = 0; k < nk; ++k) {
    __builtin_amdgcn_s_waitcnt(WAIT);
    __builtin_amdgcn_s_barrier();
    issue(min(k + STAGES - 1, nk - 1), (k + STAGES - 1) % STAGES);  // into the buffer read at k - 1
    compute(k % STAGES);
  }
  __builtin_amdgcn_s_waitcnt(0);

  // lane l stores the 8 columns 8 * ((l + 64 q) % UPR) of its wave's tile in pass q, for every
  // row: their weight scales and bias are fetched once, here, and land while the tables and the
  // first rows are staged
  constexpr int UPR = TN / 8;
  constexpr int NBQ = (64 % UPR) == 0 ? 1 : 2;  // distinct column sets among the passes (TN <= 64)
  static_assert(UPR <= 8, "two passes per 16-row group at most");
  const bool add_bias = e.bias && e.kind != OASIS_EPI_PARTIAL_F32;
  f32x4 hs[NBQ][2], hb[NBQ][2];
#pragma unroll
  for (int q = 0; q < NBQ; ++q) {
    const int gn = min(n0 + wn * TN + ((lane + 64 * q) % UPR) * 8, N - 8);
    hs[q][0] = *reinterpret_cast<const f32x4*>(wscale + gn);
    hs[q][1] = *reinterpret_cast<const f32x4*>(wscale + gn + 4);
    hb[q][0] = hb[q][1] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (add_bias) {
      hb[q][0] = *reinterpret_cast<const f32x4*>(e.bias + gn);
      hb[q][1] = *reinterpret_cast<const f32x4*>(e.bias + gn + 4);
    }
  }
  __syncthreads();

  // QKV rotation tables to LDS (above the epilogue staging) when they fit
  float* tab = reinterpret_cast<float*>(smem + EPI_BYTES);
  const int tab_rows = rope_lds_rows(e, M, SMEM - EPI_BYTES);
  if (tab_rows) {
    rope_to_lds(e, tab, tab_rows, tid, NW * 64);
    __syncthreads();
  }
  // QKV + RoPE + head split: the lane's column decisions once, its rows stepped per group
  constexpr bool QKV = KIND == OASIS_EPI_QKV_ROPE;
  QkvRows<(16 * UPR + 63) / 64> qkv;
  if constexpr (QKV) qkv.init(e, lane, UPR, n0 + wn * TN, m0 + wm * TM);
  // residual kinds: x (and gate) fetched a 16-row group ahead
  constexpr bool RES = KIND == OASIS_EPI_GATED_RES || KIND == OASIS_EPI_RESIDUAL;
  ResAhead<UPR, RES ? KIND : OASIS_EPI_RESIDUAL> res;
  if constexpr (RES) res.fetch(e, lane, m0 + wm * TM, n0 + wn * TN, M, N, 0);
  // lanes 4i..4i+3 cover one aligned 32-column block when TN % 32 == 0 (the host checks it for
  // the GELU_TANH_FP8 epilogue)
  float* st = reinterpret_cast<float*>(smem) + wave * 16 * EP;
#pragma unroll
  for (int i = 0; i < FM; ++i) {
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) st[(g * 4 + r) * EP + j * 16 + lr] = acc[i][j][r];
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    if constexpr (RES) {
      if (i + 1 < FM) res.fetch(e, lane, m0 + wm * TM + (i + 1) * 16, n0 + wn * TN, M, N, (i + 1) & 1);
#pragma unroll
      for (int q = 0; q < res.UPL; ++q) {
        const int r = res.row(lane, q), c8 = res.col(lane, q);
        const int gm = m0 + wm * TM + i * 16 + r, gn = n0 + wn * TN + c8;
        if (!res.live(lane, q) || gm >= M || gn >= N) continue;
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(st + r * EP + c8);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(st + r * EP + c8 + 4);
        const bool q1 = q > 0 && NBQ > 1;
        const f32x4 s0 = q1 ? hs[NBQ - 1][0] : hs[0][0], s1 = q1 ? hs[NBQ - 1][1] : hs[0][1];
        const f32x4 b0 = q1 ? hb[NBQ - 1][0] : hb[0][0], b1 = q1 ? hb[NBQ - 1][1] : hb[0][1];
        float v[8];
        scale_bias8(c0, c1, s0, s1, b0, b1, v);
        res.store(e, q, i & 1, gm, gn, v);
      }
    }
    for (int u = lane; !RES && u < 16 * UPR; u += 64) {
      const int r = u / UPR, c8 = (u - r * UPR) * 8;
      const int gm = m0 + wm * TM + i * 16 + r, gn = n0 + wn * TN + c8;
      if (gm < M && gn < N) {
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(st + r * EP + c8);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(st + r * EP + c8 + 4);
        const bool q1 = NBQ > 1 && u >= 64;
        const f32x4 s0 = q1 ? hs[NBQ - 1][0] : hs[0][0], s1 = q1 ? hs[NBQ - 1][1] : hs[0][1];
        const f32x4 b0 = q1 ? hb[NBQ - 1][0] : hb[0][0], b1 = q1 ? hb[NBQ - 1][1] : hb[0][1];
        float v[8];
        scale_bias8(c0, c1, s0, s1, b0, b1, v);
        if constexpr (QKV) {
          qkv.store(e, u >> 6, v, tab, tab_rows);
        } else if (KIND == OASIS_EPI_PARTIAL_F32 || (KIND < 0 && e.kind == OASIS_EPI_PARTIAL_F32)) {
          float* d = e.out_f32 + (int64_t)split * e.split_stride + (int64_t)gm * e.ld_out + gn;
          *reinterpret_cast<f32x4*>(d) = f32x4{v[0], v[1], v[2], v[3]};
          *reinterpret_cast<f32x4*>(d + 4) = f32x4{v[4], v[5], v[6], v[7]};
        } else {
          epilogue8(e, gm, gn, v, tab_rows ? tab : nullptr, tab_rows, false, KIND);
        }
      }
    }
    if constexpr (QKV) qkv.advance(e);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

typedef hipError_t (*launch8_fn)(const void*, int64_t, const uint8_t*, int64_t, const uint8_t*, int64_t,
                                 const float*, int, int, int, int, const Epi&, hipStream_t);

template <int BM, int BN, int WM, int WN, int STAGES, bool AQ>
hipError_t launch8(const void* A, int64_t lda, const uint8_t* As, int64_t lds, const uint8_t* B, int64_t ldb,
                   const float* ws, int M, int N, int K, int splits, const Epi& e, hipStream_t s) {
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_fp8_kernel<BM, BN, WM, WN, STAGES, AQ>), dim3(Mt * Nt * splits), dim3(256), 0, s, A,
                     lda, As, lds, B, ldb, ws, M, N, K, splits, e);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int STAGES = 2>
hipError_t launch8_big(const void* A, int64_t lda, const uint8_t* As, int64_t lds, const uint8_t* B, int64_t ldb,
                       const float* ws, int M, int N, int K, int splits, const Epi& e, hipStream_t s) {
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  if (e.kind == OASIS_EPI_QKV_ROPE)
    hipLaunchKernelGGL((gemm_fp8_big_kernel<BM, BN, WM, WN, OASIS_EPI_QKV_ROPE, STAGES>), dim3(Mt * Nt * splits),
                       dim3(WM * WN * 64), 0, s, static_cast<const uint8_t*>(A), lda, As, lds, B, ldb, ws, M, N, K,
                       splits, e);
  else if (e.kind == OASIS_EPI_GELU_TANH_FP8)
    hipLaunchKernelGGL((gemm_fp8_big_kernel<BM, BN, WM, WN, OASIS_EPI_GELU_TANH_FP8, STAGES>), dim3(Mt * Nt * splits),
                       dim3(WM * WN * 64), 0, s, static_cast<const uint8_t*>(A), lda, As, lds, B, ldb, ws, M, N, K,
                       splits, e);
  else if (e.kind == OASIS_EPI_PARTIAL_F32)
    hipLaunchKernelGGL((gemm_fp8_big_kernel<BM, BN, WM, WN, OASIS_EPI_PARTIAL_F32, STAGES>), dim3(Mt * Nt * splits),
                       dim3(WM * WN * 64), 0, s, static_cast<const uint8_t*>(A), lda, As, lds, B, ldb, ws, M, N, K,
                       splits, e);
  else if (e.kind == OASIS_EPI_GATED_RES)
    hipLaunchKernelGGL((gemm_fp8_big_kernel<BM, BN, WM, WN, OASIS_EPI_GATED_RES, STAGES>), dim3(Mt * Nt * splits),
                       dim3(WM * WN * 64), 0, s, static_cast<const uint8_t*>(A), lda, As, lds, B, ldb, ws, M, N, K,
                       splits, e);
  else if (e.kind == OASIS_EPI_RESIDUAL)
    hipLaunchKernelGGL((gemm_fp8_big_kernel<BM, BN, WM, WN, OASIS_EPI_RESIDUAL, STAGES>), dim3(Mt * Nt * splits),
                       dim3(WM * WN * 64), 0, s, static_cast<const uint8_t*>(A), lda, As, lds, B, ldb, ws, M, N, K,
                       splits, e);
  else
    hipLaunchKernelGGL((gemm_fp8_big_kernel<BM, BN, WM, WN, -1, STAGES>), dim3(Mt * Nt * splits), dim3(WM * WN * 64), 0, s,
                       static_cast<const uint8_t*>(A), lda, As, lds, B, ldb, ws, M, N, K, splits, e);
  return hipGetLastError();
}

struct Tile8 {
  int bm, bn, stages;
  launch8_fn fn, fn_single;        // bf16 A (null: fp8 A only)
  launch8_fn fn_q, fn_q_single;    // fp8 A blocks
  int no_fp8_epi;                  // 1: its epilogue lanes do not cover aligned 32-column blocks
};
#define OASIS_T8(BM, BN, WM, WN)                                                                       \
  {BM, BN, 2, launch8<BM, BN, WM, WN, 2, false>, launch8<BM, BN, WM, WN, 1, false>,                   \
   launch8<BM, BN, WM, WN, 2, true>, launch8<BM, BN, WM, WN, 1, true>, 0}
#define OASIS_T8_BIG(BM, BN, WM, WN, NO_FP8_EPI, ST) \
  {BM, BN, 1, nullptr, nullptr, launch8_big<BM, BN, WM, WN, ST>, launch8_big<BM, BN, WM, WN, ST>, NO_FP8_EPI}
const Tile8 kTiles8[] = {
    OASIS_T8(128, 128, 2, 2),              // 0
    OASIS_T8(128, 64, 2, 2),               // 1
    OASIS_T8(64, 128, 2, 2),               // 2
    OASIS_T8(64, 64, 2, 2),                // 3
    OASIS_T8(32, 64, 1, 4),                // 4
    OASIS_T8_BIG(288, 256, 2, 4, 0, 2),    // 5  (fp8 A only; two stages)
    OASIS_T8_BIG(288, 192, 2, 4, 1, 2),    // 6
    OASIS_T8_BIG(288, 128, 2, 4, 0, 2),    // 7
    OASIS_T8_BIG(144, 128, 3, 2, 0, 2),    // 8  (N = 1024 unsplit at 4608 tokens: 256 tiles)
    OASIS_T8_BIG(288, 64, 2, 4, 1, 2),     // 9
    OASIS_T8_BIG(144, 128, 3, 2, 0, 3),    // 10 (three stages)
    OASIS_T8_BIG(144, 128, 3, 2, 0, 4),    // 11 (four stages)
};
#undef OASIS_T8
#undef OASIS_T8_BIG
constexpr int kNumTiles8 = sizeof(kTiles8) / sizeof(kTiles8[0]);

// Default tile per shape, from sweeps of the DiT projections at M = 4608 on MI355X: with fp8 A
// from 2048 tokens up the 8-wave 288-row tiles (as the bf16 GEMM picks them).
int auto_tile8(int64_t M, int64_t N, bool aq, int kind) {
  if (M >= 2048 && aq) return large_token_tile(M, N, kind != OASIS_EPI_GELU_TANH_FP8, 5, 6, 7);
  if (M >= 2048) return 2;
  if (M >= 256) return 3;
  return 4;
}

// Per-row quantization of a bf16 [N, K] weight: scale[n] = max|W[n, :]| / 448,
// q[n, k] = round_e4m3(W[n, k] / scale[n]) (round to nearest even). One wave per row.
__global__ __launch_bounds__(256) void quant_rows_kernel(const bf16* __restrict__ W, int64_t N, int64_t K,
                                                         uint8_t* __restrict__ q, float* __restrict__ scale) {
  const int64_t n = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  if (n >= N) return;
  const bf16* w = W + n * K;
  float amax = 0.f;
  for (int64_t k = lane * 8; k < K; k += 512) {
    const bf16x8 h = *reinterpret_cast<const bf16x8*>(w + k);
#pragma unroll
    for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf((float)h[j]));
  }
  amax = wave_max(amax);
  const float s = amax > 0.f ? amax / 448.0f : 1.0f;
  if (lane == 0) scale[n] = s;
  for (int64_t k = lane * 8; k < K; k += 512) {
    const bf16x8 h = *reinterpret_cast<const bf16x8*>(w + k);
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32((float)h[0] / s, (float)h[1] / s, 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32((float)h[2] / s, (float)h[3] / s, lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32((float)h[4] / s, (float)h[5] / s, 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32((float)h[6] / s, (float)h[7] / s, hi, true);
    *reinterpret_cast<uint2*>(q + n * K + k) = make_uint2((unsigned)lo, (unsigned)hi);
  }
}

// bf16 [M, K] activations -> e4m3 blocks of 32 along K with e8m0 scales [M, K/32].
// Each thread converts 8 consecutive values; lanes 4i..4i+3 share one block.
__global__ __launch_bounds__(256) void quant_act_kernel(const bf16* __restrict__ x, int64_t ldx, int64_t M, int64_t K,
                                                        uint8_t* __restrict__ q, int64_t ldq,
                                                        uint8_t* __restrict__ sc, int64_t lds) {
  const int64_t cpr = K / 8;  // 8-value chunks per row
  const int64_t n = M * cpr;
  const int64_t step = (int64_t)gridDim.x * blockDim.x;  // a multiple of 4: groups never straddle
  for (int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; c - (threadIdx.x & 3) < n; c += step) {
    const bool live = c < n;
    const int64_t cc = live ? c : n - 1;
    const int64_t m = cc / cpr, k = (cc - m * cpr) * 8;
    int sb;
    const uint2 v = quant8(*reinterpret_cast<const i32x4*>(x + m * ldx + k), &sb);
    if (live) {
      *reinterpret_cast<uint2*>(q + m * ldq + k) = v;
      if ((k & 31) == 0) sc[m * lds + k / 32] = (uint8_t)sb;
    }
  }
}

}  // namespace

namespace oasis {

int gemm_fp8_launch(const void* A, int64_t lda, const uint8_t* A_scale, int64_t lds, const uint8_t* B, int64_t ldb,
                    const float* w_scale, int64_t M, int64_t N, int64_t K, const oasis_epilogue_t& ex, int tile,
                    int splits, hipStream_t s) {
  const bool aq = A_scale != nullptr;
  OASIS_REQUIRE(A && B && w_scale, OASIS_ERR_NULL, "gemm_fp8: null operand");
  OASIS_REQUIRE(ex.kind != OASIS_EPI_GATED_RES_LN && ex.kind != OASIS_EPI_GELU_TANH_LN, OASIS_ERR_ARG,
                "gemm_fp8: epilogue kind %d runs on oasis_gemm_bf16_frag only", ex.kind);
  OASIS_REQUIRE(aligned16(A) && aligned16(B) && aligned16(w_scale) && (reinterpret_cast<uintptr_t>(A_scale) & 3) == 0,
                OASIS_ERR_ARG, "gemm_fp8: A, B and w_scale must be 16-byte aligned, A_scale 4-byte aligned");
  OASIS_REQUIRE(!aq || (lds >= K / 32 && lds % 4 == 0 && lda % 16 == 0), OASIS_ERR_SHAPE,
                "gemm_fp8: fp8 A needs lda %% 16 == 0 and lds >= K/32, lds %% 4 == 0");
  OASIS_REQUIRE(M > 0 && N > 0 && K > 0 && M < (1ll << 31) && N < (1ll << 31), OASIS_ERR_SHAPE,
                "gemm_fp8: bad shape M=%lld N=%lld K=%lld", (long long)M, (long long)N, (long long)K);
  OASIS_REQUIRE(K % BK8 == 0, OASIS_ERR_SHAPE, "gemm_fp8: K=%lld must be a multiple of 128", (long long)K);
  OASIS_REQUIRE(N % 8 == 0, OASIS_ERR_SHAPE, "gemm_fp8: N=%lld must be a multiple of 8", (long long)N);
  OASIS_REQUIRE(lda % 8 == 0 && ldb % 16 == 0 && lda >= K && ldb >= K, OASIS_ERR_SHAPE,
                "gemm_fp8: need lda %% 8 == 0, ldb %% 16 == 0, both >= K");
  // the kernels address a tile's rows by 32-bit byte offsets from its first row
  OASIS_REQUIRE(lda < (1ll << 22) && ldb < (1ll << 22), OASIS_ERR_SHAPE, "gemm_fp8: lda/ldb must be below 2^22");
  OASIS_REQUIRE(splits >= 1 && (K / BK8) % splits == 0, OASIS_ERR_SHAPE, "gemm_fp8: splits=%d must divide K/128",
                splits);
  const Epi e = to_epi(ex);
  if (const int rc = check_epilogue(e, M, N, splits)) return rc;
  if (tile < 0) tile = auto_tile8(M, N, aq, e.kind);
  OASIS_REQUIRE(tile < kNumTiles8, OASIS_ERR_ARG, "gemm_fp8: tile config %d out of range", tile);
  const Tile8& t = kTiles8[tile];
  OASIS_REQUIRE(!(t.no_fp8_epi && e.kind == OASIS_EPI_GELU_TANH_FP8), OASIS_ERR_ARG,
                "gemm_fp8: tile config %d cannot run the GELU_TANH_FP8 epilogue", tile);
  OASIS_REQUIRE(aq || t.fn, OASIS_ERR_ARG, "gemm_fp8: tile config %d needs A as fp8 blocks", tile);
  const bool ring = (K / BK8 / splits) % t.stages == 0;
  const launch8_fn fn = aq ? (ring ? t.fn_q : t.fn_q_single) : (ring ? t.fn : t.fn_single);
  const hipError_t err = fn(A, lda, A_scale, lds, B, ldb, w_scale, (int)M, (int)N, (int)K, splits, e, s);
  if (err != hipSuccess) {
    set_error("gemm_fp8 launch failed: %s", hipGetErrorString(err));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

}  // namespace oasis

extern "C" int oasis_gemm_fp8(const void* A, int64_t lda, const void* B, int64_t ldb, const float* w_scale, int64_t M,
                              int64_t N, int64_t K, const oasis_epilogue_t* epi, int tile, int splits,
                              oasis_stream_t stream) {
  OASIS_REQUIRE(epi, OASIS_ERR_NULL, "gemm_fp8: null epilogue");
  return oasis::gemm_fp8_launch(A, lda, nullptr, 0, static_cast<const uint8_t*>(B), ldb, w_scale, M, N, K, *epi, tile,
                                splits, static_cast<hipStream_t>(stream));
}

extern "C" int oasis_gemm_fp8_a8(const void* A8, int64_t lda, const void* A_scale, int64_t lds, const void* B,
                                 int64_t ldb, const float* w_scale, int64_t M, int64_t N, int64_t K,
                                 const oasis_epilogue_t* epi, int tile, int splits, oasis_stream_t stream) {
  OASIS_REQUIRE(epi, OASIS_ERR_NULL, "gemm_fp8_a8: null epilogue");
  OASIS_REQUIRE(A_scale, OASIS_ERR_NULL, "gemm_fp8_a8: null A scales");
  return oasis::gemm_fp8_launch(A8, lda, static_cast<const uint8_t*>(A_scale), lds, static_cast<const uint8_t*>(B),
                                ldb, w_scale, M, N, K, *epi, tile, splits, static_cast<hipStream_t>(stream));
}

extern "C" int oasis_quantize_act_fp8(const void* x, int64_t ldx, int64_t M, int64_t K, void* q, int64_t ldq,
                                      void* scale, int64_t lds, oasis_stream_t stream) {
  OASIS_REQUIRE(x && q && scale, OASIS_ERR_NULL, "quantize_act_fp8: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, x) && oasis_aligned(8, q), OASIS_ERR_ARG, "quantize_act_fp8: x must be 16-byte, q 8-byte aligned");
  OASIS_REQUIRE(M > 0 && K > 0 && K % 32 == 0 && ldx >= K && ldx % 8 == 0 && ldq >= K && ldq % 8 == 0 && lds >= K / 32,
                OASIS_ERR_SHAPE, "quantize_act_fp8: need K %% 32 == 0, ldx/ldq >= K (multiples of 8), lds >= K/32");
  const int64_t chunks = M * (K / 8);
  int64_t blocks = (chunks + 255) / 256;
  if (blocks > 4096) blocks = 4096;
  hipLaunchKernelGGL(quant_act_kernel, dim3((unsigned)blocks), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(x), ldx, M, K, static_cast<uint8_t*>(q), ldq,
                     static_cast<uint8_t*>(scale), lds);
  return oasis::check_launch("quantize_act_fp8");
}

extern "C" int oasis_quantize_fp8_rows(const void* W, int64_t N, int64_t K, void* q, float* scale,
                                       oasis_stream_t stream) {
  OASIS_REQUIRE(W && q && scale, OASIS_ERR_NULL, "quantize_fp8_rows: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, W) && oasis_aligned(8, q), OASIS_ERR_ARG, "quantize_fp8_rows: W must be 16-byte, q 8-byte aligned");
  OASIS_REQUIRE(N > 0 && K > 0 && K % 8 == 0 && N <= (1ll << 30), OASIS_ERR_SHAPE,
                "quantize_fp8_rows: need N > 0 and K a positive multiple of 8");
  hipLaunchKernelGGL(quant_rows_kernel, dim3((unsigned)((N + 3) / 4)), dim3(256), 0, static_cast<hipStream_t>(stream),
                     static_cast<const bf16*>(W), N, K, static_cast<uint8_t*>(q), scale);
  return oasis::check_launch("quantize_fp8_rows");
}
