// bf16 MFMA GEMM for gfx950 with fused epilogues.
//
//   acc[M,N] = A[M,K] @ B[N,K]^T, A = activations (bf16, row-major), B = weights in
//   the nn.Linear layout [out, in] (bf16), fp32 accumulation, then one epilogue
//   (bias, tanh/erf GELU, gated residual into the fp32 stream, RoPE + head split,
//   VAE unpatchify, split-K slices) applied on the way out.
//
// Kernels (v_mfma_f32_16x16x32_bf16 throughout; K in 64-wide tiles):
//   - gemm_lds_kernel: 4 waves, the K tiles copied global -> LDS by the memory pipeline itself
//     (global_load_lds_dwordx4) into a ring of STAGES tiles; small tiles for the split-K slices
//     and the QKV + RoPE product at 144 / 288 tokens.
//   - gemm_big_kernel: the same ring with a grouped tile order and a per-wave staged epilogue, on
//     4-, 6- and 8-wave tiles: the MLP products, every VAE projection, and the 8-wave 288-row
//     tiles from 2048 tokens up.
//   - gemm_wave_kernel: 4 waves split each workgroup's K slice four ways, each over its own LDS
//     ring with no workgroup barrier in the K loop; the default below 320 tokens (QKV + RoPE, O,
//     FC1, FC2) and for the VAE's O projection.
//   - gemm_bf16_kernel: global -> registers -> LDS, for the reference-surface oasis_linear with
//     its [K, N] weight layout (the weights transposed into LDS).
// After the K loop the fp32 tile is staged through LDS so each thread handles 8 consecutive
// columns of one row: coalesced 16/32-byte stores and in-register RoPE pair swaps.
//
// Workgroup -> tile order is XCD-aware: MI355X dispatches workgroup i to XCD i % 8,
// so ids are remapped such that every M tile of one weight column block lands on the
// same XCD; the weight block is then fetched from HBM once into that XCD's L2.
#include <string.h>

#include <algorithm>

#include "gemm_epilogue.h"

namespace {

constexpr int BK = 64;            // K granularity every configuration supports

// BKN = false: B is [N, K] (weights as stored by this library); true: B is [K, N]
// (the reference's transposed weight layout, used by the linear_k32 surface only).
// STAGES K-tiles are in flight per workgroup: a register ring of STAGES global-load
// slots feeds a double-buffered LDS tile pair. With `splits` > 1 the K range is cut
// into equal slices, one per workgroup, and the epilogue must be PARTIAL_F32.
template <int BM, int BN, int WM, int WN, int STAGES, bool BKN, int BKT>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(const bf16* __restrict__ A, int64_t lda,
                                                        const bf16* __restrict__ B, int64_t ldb,
                                                        int M, int N, int K, int splits, Epi e) {
  static_assert(WM * WN == 4, "4 waves");
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  static_assert(FM * 16 == TM && FN * 16 == TN, "wave tile must be a multiple of 16");
  constexpr int BK = BKT;                  // K per pipeline step
  constexpr int LDS_PITCH = BK + 8;        // bf16 per LDS row (16 B pad: conflict-free b128 reads)
  constexpr int CPR = BK / 8;              // 16-byte chunks per tile row
  constexpr int A_CHUNKS = BM * CPR;       // 16-byte chunks per A tile
  constexpr int B_CHUNKS = BN * CPR;
  // every thread loads whole chunks: no per-thread guards, so the compiler can keep
  // STAGES tiles of loads in flight (a divergent guard forces a full vmcnt(0) wait)
  static_assert(A_CHUNKS % 256 == 0 && B_CHUNKS % 256 == 0, "BM and BN must be multiples of 32");
  constexpr int A_PER = A_CHUNKS / 256;
  constexpr int B_PER = B_CHUNKS / 256;
  constexpr int AB_BYTES = 2 * (BM + BN) * LDS_PITCH * 2;
  constexpr int C_PITCH = BN + 4;
  constexpr int C_BYTES = BM * C_PITCH * 4;
  constexpr int SMEM = AB_BYTES > C_BYTES ? AB_BYTES : C_BYTES;
  __shared__ __attribute__((aligned(16))) char smem[SMEM];
  bf16* As = reinterpret_cast<bf16*>(smem);                    // [2][BM][LDS_PITCH]
  bf16* Bs = As + 2 * BM * LDS_PITCH;                          // [2][BN][LDS_PITCH]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave % WM, wn = wave / WM;
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  // (n tile, split, m tile) with m fastest: consecutive ids share one weight slice
  const int pid = xcd_remap(blockIdx.x, Mt * Nt * splits);
  const int mt = pid % Mt;
  const int rest = pid / Mt;
  const int split = rest % splits, nt = rest / splits;
  const int m0 = mt * BM, n0 = nt * BN;
  const int nk = K / BK / splits;  // the host guarantees nk % STAGES == 0
  const int kb = split * nk * BK;

  const bf16* a_src[A_PER];
  int a_dst[A_PER];
#pragma unroll
  for (int i = 0; i < A_PER; ++i) {
    const int c = tid + i * 256;
    const int row = c / CPR, col = (c % CPR) * 8;
    const int gr = min(m0 + row, M - 1);
    a_src[i] = A + (int64_t)gr * lda + kb + col;
    a_dst[i] = row * LDS_PITCH + col;
  }
  const bf16* b_src[B_PER];
  int b_dst[B_PER];
#pragma unroll
  for (int i = 0; i < B_PER; ++i) {
    const int c = tid + i * 256;
    if (!BKN) {
      const int row = c / CPR, col = (c % CPR) * 8;
      const int gr = min(n0 + row, N - 1);
      b_src[i] = B + (int64_t)gr * ldb + kb + col;
      b_dst[i] = row * LDS_PITCH + col;
    } else {  // chunk = 8 consecutive n of one k row; stored transposed into [n][k]
      const int krow = c / (BN / 8), nc = (c % (BN / 8)) * 8;
      const int gn = min(n0 + nc, N - 8);
      b_src[i] = B + (int64_t)(kb + krow) * ldb + gn;
      b_dst[i] = nc * LDS_PITCH + krow;
    }
  }

  i32x4 ra[STAGES][A_PER], rb[STAGES][B_PER];
  auto gload = [&](int slot, int kt) {
    const int64_t ka = (int64_t)kt * BK;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) ra[slot][i] = *reinterpret_cast<const i32x4*>(a_src[i] + ka);
#pragma unroll
    for (int i = 0; i < B_PER; ++i)
      rb[slot][i] = *reinterpret_cast<const i32x4*>(b_src[i] + (BKN ? ka * ldb : ka));
  };
  auto lstore = [&](int slot, int buf) {
    bf16* as = As + buf * BM * LDS_PITCH;
    bf16* bs = Bs + buf * BN * LDS_PITCH;
#pragma unroll
    for (int i = 0; i < A_PER; ++i) *reinterpret_cast<i32x4*>(as + a_dst[i]) = ra[slot][i];
#pragma unroll
    for (int i = 0; i < B_PER; ++i) {
      if (!BKN) {
        *reinterpret_cast<i32x4*>(bs + b_dst[i]) = rb[slot][i];
      } else {
        const bf16x8 t = __builtin_bit_cast(bf16x8, rb[slot][i]);
#pragma unroll
        for (int j = 0; j < 8; ++j) bs[b_dst[i] + j * LDS_PITCH] = t[j];
      }
    }
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, lk = (lane >> 4) * 8;
  auto compute = [&](int buf) {
    const bf16* as = As + buf * BM * LDS_PITCH + (wm * TM + lr) * LDS_PITCH + lk;
    const bf16* bs = Bs + buf * BN * LDS_PITCH + (wn * TN + lr) * LDS_PITCH + lk;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(as + i * 16 * LDS_PITCH + ks * 32);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(bs + j * 16 * LDS_PITCH + ks * 32);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(af[i], bfr[j], acc[i][j]);
    }
  };

  // Prologue: tiles 0..STAGES-1 in flight, tile 0 in LDS. Tile indices past the end are
  // clamped to the last tile (a redundant L2 hit) instead of branched around, so the
  // loop body is straight-line and the waits before each LDS store count only the
  // STAGES-1 younger tiles.
#pragma unroll
  for (int s = 0; s < STAGES; ++s) gload(s, min(s, nk - 1));
  lstore(0, 0);
  __syncthreads();
  for (int k0 = 0; k0 < nk; k0 += STAGES) {
#pragma unroll
    for (int s = 0; s < STAGES; ++s) {
      const int k = k0 + s;
      gload(s, min(k + STAGES, nk - 1));     // slot s held tile k, already in LDS
      compute(k & 1);
      lstore((s + 1) % STAGES, (k + 1) & 1);  // tile k+1 (a copy of the last tile at the end)
      __syncthreads();
    }
  }

  // stage the fp32 tile through LDS (the A/B ring is free after the last barrier)
  float* Cs = reinterpret_cast<float*>(smem);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        Cs[(wm * TM + i * 16 + (lane >> 4) * 4 + r) * C_PITCH + wn * TN + j * 16 + lr] = acc[i][j][r];
  __syncthreads();

  constexpr int UNITS = BM * (BN / 8);
  for (int u = tid; u < UNITS; u += 256) {
    const int r = u / (BN / 8), c8 = (u % (BN / 8)) * 8;
    const int gm = m0 + r, gn = n0 + c8;
    if (gm >= M || gn >= N) continue;
    float v[8];
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(Cs + r * C_PITCH + c8);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(Cs + r * C_PITCH + c8 + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = c0[j];
      v[j + 4] = c1[j];
    }
    if (e.kind == OASIS_EPI_PARTIAL_F32) {
      float* d = e.out_f32 + (int64_t)split * e.split_stride + (int64_t)gm * e.ld_out + gn;
      *reinterpret_cast<f32x4*>(d) = c0;
      *reinterpret_cast<f32x4*>(d + 4) = c1;
    } else {
      epilogue8(e, gm, gn, v);
    }
  }
}

// Same product with the global -> LDS copies done by the memory pipeline itself
// (global_load_lds_dwordx4: each lane's 16 bytes land at LDS base + 16 * lane), so tiles
// take no VGPRs or LDS-store instructions in flight and STAGES K tiles can be queued per
// workgroup. LDS rows are unpadded 128-byte rows of 16-byte chunks stored XOR-swizzled
// (chunk c of row r at slot c ^ ((r >> 1) & 7)), which keeps the 16-row MFMA fragment
// reads conflict-free. One wave instruction fills 8 rows; the A rows come first.
template <int BM, int BN, int WM, int WN, int STAGES>
__global__ __launch_bounds__(256) void gemm_lds_kernel(const bf16* __restrict__ A, int64_t lda,
                                                       const bf16* __restrict__ B, int64_t ldb, int M, int N,
                                                       int K, int splits, Epi e) {
  static_assert(WM * WN == 4, "4 waves");
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  static_assert(FM * 16 == TM && FN * 16 == TN, "wave tile must be a multiple of 16");
  constexpr int ROWB = 128;                     // bytes per LDS row: 64 bf16 of K
  constexpr int NBLK = (BM + BN) / 8;           // 1 KB blocks (8 rows) per stage
  static_assert(BM % 8 == 0 && BN % 8 == 0, "whole 8-row blocks");
  // loads per wave per stage; when NBLK % 4 != 0 the last wave re-loads the last block (same
  // bytes to the same LDS slots), so every wave waits on the same vmcnt
  constexpr int LPW = (NBLK + 3) / 4;
  constexpr int STAGE_BYTES = (BM + BN) * ROWB;
  constexpr int RING = STAGES * STAGE_BYTES;
  constexpr int C_PITCH = BN + 4;
  constexpr int C_BYTES = BM * C_PITCH * 4;
  constexpr int SMEM = RING > C_BYTES ? RING : C_BYTES;
  static_assert(STAGES >= 2 && (STAGES - 2) * LPW <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  // the wave index read back as a scalar, so that the load bases built from it stay in SGPRs
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  const int pid = xcd_remap(blockIdx.x, Mt * Nt * splits);
  const int mt = pid % Mt;
  const int rest = pid / Mt;
  const int split = rest % splits, nt = rest / splits;
  const int m0 = mt * BM, n0 = nt * BN;
  const int nk = K / 64 / splits;
  const int kb = split * nk * 64;

  // this lane's source in each of its LPW blocks: row r = 8 * blk + lane / 8 of the A|B stack,
  // slot lane % 8 holds K chunk (lane % 8) ^ ((r >> 1) & 7); buffer loads from the tile's first
  // A row / weight row (scalar base, K tile as scalar offset, 32-bit lane offset)
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
    off[u] = from_a[u] ? (uint32_t)(((int64_t)(min(m0 + r, M - 1) - m0) * lda + c * 8) * 2)
                       : (uint32_t)(((int64_t)(min(n0 + r - BM, N - 1) - n0) * ldb + c * 8) * 2);
    dst[u] = blk * 1024;
  }
  auto issue = [&](int kt, int buf) {
    char* base = smem + buf * STAGE_BYTES;
#pragma unroll
    for (int u = 0; u < LPW; ++u) buffer_load_lds16(from_a[u] ? Ars : Brs, off[u], kt * 128, base + dst[u]);
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
      const int c = ks * 4 + g;  // 16-byte K chunk of this lane's 8 values
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
      for (int r = 0; r < 4; ++r)
        Cs[(wm * TM + i * 16 + g * 4 + r) * C_PITCH + wn * TN + j * 16 + lr] = acc[i][j][r];
  __syncthreads();

  constexpr int UNITS = BM * (BN / 8);
  for (int u = tid; u < UNITS; u += 256) {
    const int r = u / (BN / 8), c8 = (u % (BN / 8)) * 8;
    const int gm = m0 + r, gn = n0 + c8;
    if (gm >= M || gn >= N) continue;
    float v[8];
    const f32x4 c0 = *reinterpret_cast<const f32x4*>(Cs + r * C_PITCH + c8);
    const f32x4 c1 = *reinterpret_cast<const f32x4*>(Cs + r * C_PITCH + c8 + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] = c0[j];
      v[j + 4] = c1[j];
    }
    if (e.kind == OASIS_EPI_PARTIAL_F32) {
      float* d = e.out_f32 + (int64_t)split * e.split_stride + (int64_t)gm * e.ld_out + gn;
      *reinterpret_cast<f32x4*>(d) = c0;
      *reinterpret_cast<f32x4*>(d + 4) = c1;
    } else {
      epilogue8(e, gm, gn, v);
    }
  }
}

// Large-token variant (2048+ tokens: many frames or streams per pass): 8 waves (2 per SIMD)
// share one tall tile such as 288 x 256 (two 144-token frames by 256 output channels), so
// each K tile of 64 brings 4.7 MFLOP per 68 KB staged, and a 4608-token projection is one
// round of 256 workgroups. Same direct-to-LDS ring and swizzle as gemm_lds_kernel (two
// stages fit in LDS). Tiles are ordered (split, groups of GN n tiles, m, n within group) so
// an XCD's consecutive ids cover a compact block of tiles: each XCD's L2 then holds a few
// rows of A and a few weight slices instead of every row of A.
// The epilogue stages 16 rows of a wave's tile at a time in LDS owned by that wave alone.

template <int BM, int BN, int WM, int WN, int STAGES, int GN = 8, int KIND = -1>
__global__ __launch_bounds__(WM * WN * 64) void gemm_big_kernel(const bf16* __restrict__ A, int64_t lda,
                                                               const bf16* __restrict__ B, int64_t ldb, int M,
                                                               int N, int K, int splits, Epi e) {
  constexpr int NW = WM * WN;
  constexpr int TM = BM / WM, TN = BN / WN;
  constexpr int FM = TM / 16, FN = TN / 16;
  static_assert(FM * 16 == TM && FN * 16 == TN, "wave tile must be a multiple of 16");
  constexpr int ROWB = 128;
  constexpr int NBLK = (BM + BN) / 8;
  static_assert(BM % 8 == 0 && BN % 8 == 0, "whole 8-row blocks");
  constexpr int LPW = (NBLK + NW - 1) / NW;
  constexpr int STAGE_BYTES = (BM + BN) * ROWB;
  constexpr int RING = STAGES * STAGE_BYTES;
  constexpr int EP = TN + 4;  // fp32 pitch of a wave's 16-row staging block
  constexpr int EPI_BYTES = NW * 16 * EP * 4;
  constexpr int SMEM = RING > EPI_BYTES ? RING : EPI_BYTES;
  static_assert(SMEM <= 160 * 1024, "LDS");
  static_assert(STAGES >= 2 && (STAGES - 2) * LPW <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  // the wave index read back as a scalar, so that the load bases built from it stay in SGPRs
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WM, wn = wave / WM;
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  int split, mt, nt;
  grouped_tile(xcd_remap(blockIdx.x, Mt * Nt * splits), Mt, Nt, GN, split, mt, nt);
  const int m0 = mt * BM, n0 = nt * BN;
  const int nk = K / 64 / splits;
  const int kb = split * nk * 64;

  // buffer loads (as in gemm_wave_kernel): the tile's first A row / weight row as the scalar base,
  // the K tile as a scalar offset, a 32-bit lane offset below BM (BN) rows of lda (ldb)
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
    off[u] = from_a[u] ? (uint32_t)(((int64_t)(min(m0 + r, M - 1) - m0) * lda + c * 8) * 2)
                       : (uint32_t)(((int64_t)(min(n0 + r - BM, N - 1) - n0) * ldb + c * 8) * 2);
    dst[u] = blk * 1024;
  }
  auto issue = [&](int kt, int buf) {
    char* base = smem + buf * STAGE_BYTES;
#pragma unroll
    for (int u = 0; u < LPW; ++u) buffer_load_lds16(from_a[u] ? Ars : Brs, off[u], kt * 128, base + dst[u]);
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

  constexpr int VM = (STAGES - 2) * LPW;
  constexpr int WAIT = (VM & 15) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8);
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s) issue(min(s, nk - 1), s);
  for (int k = 0; k < nk; ++k) {
    __builtin_amdgcn_s_waitcnt(WAIT);
    __builtin_amdgcn_s_barrier();
    issue(min(k + STAGES - 1, nk - 1), (k + STAGES - 1) % STAGES);
    compute(k % STAGES);
  }
  __builtin_amdgcn_s_waitcnt(0);

  // The epilogue gives lane l the 8 columns 8 * ((l + 64 q) % UPR) of its wave's tile in pass q,
  // for every row: their bias is fetched once, here (a load per stored row would put a memory
  // round trip into every pass), and lands while the tables and first rows are staged.
  constexpr int UPR = TN / 8;
  constexpr int NBQ = (64 % UPR) == 0 ? 1 : 2;  // distinct column sets among the passes (TN <= 64)
  static_assert(UPR <= 8, "two passes per 16-row group at most");
  const bool add_bias = e.bias && e.kind != OASIS_EPI_PARTIAL_F32;
  f32x4 hb[NBQ][2];
#pragma unroll
  for (int q = 0; q < NBQ; ++q) {
    const int gn = min(n0 + wn * TN + ((lane + 64 * q) % UPR) * 8, N - 8);
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

  // each lane takes 8 consecutive columns of one row; lanes 4i..4i+3 cover one aligned 32-column
  // block when TN % 32 == 0 (the fp8 epilogue's shuffles rely on it; the host checks)
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
        const f32x4 b0 = q > 0 && NBQ > 1 ? hb[NBQ - 1][0] : hb[0][0];
        const f32x4 b1 = q > 0 && NBQ > 1 ? hb[NBQ - 1][1] : hb[0][1];
        const float v[8] = {c0[0] + b0[0], c0[1] + b0[1], c0[2] + b0[2], c0[3] + b0[3],
                            c1[0] + b1[0], c1[1] + b1[1], c1[2] + b1[2], c1[3] + b1[3]};
        res.store(e, q, i & 1, gm, gn, v);
      }
    }
    for (int u = lane; !RES && u < 16 * UPR; u += 64) {
      const int r = u / UPR, c8 = (u - r * UPR) * 8;
      const int gm = m0 + wm * TM + i * 16 + r, gn = n0 + wn * TN + c8;
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(st + r * EP + c8);
      const f32x4 c1 = *reinterpret_cast<const f32x4*>(st + r * EP + c8 + 4);
      if (gm < M && gn < N) {
        if (KIND == OASIS_EPI_PARTIAL_F32 || (KIND < 0 && e.kind == OASIS_EPI_PARTIAL_F32)) {
          float* d = e.out_f32 + (int64_t)split * e.split_stride + (int64_t)gm * e.ld_out + gn;
          *reinterpret_cast<f32x4*>(d) = c0;
          *reinterpret_cast<f32x4*>(d + 4) = c1;
        } else {
          const bool q1 = NBQ > 1 && u >= 64;
          const f32x4 b0 = q1 ? hb[NBQ - 1][0] : hb[0][0], b1 = q1 ? hb[NBQ - 1][1] : hb[0][1];
          float v[8] = {c0[0] + b0[0], c0[1] + b0[1], c0[2] + b0[2], c0[3] + b0[3],
                        c1[0] + b1[0], c1[1] + b1[1], c1[2] + b1[2], c1[3] + b1[3]};
          if constexpr (QKV) {
            qkv.store(e, u >> 6, v, tab, tab_rows);
          } else {
            epilogue8(e, gm, gn, v, tab_rows ? tab : nullptr, tab_rows, false, KIND);
          }
        }
      }
    }
    if constexpr (QKV) qkv.advance(e);
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }
}

// Wave-split K (below 2048 tokens): the 4 waves of a workgroup share one BM x BN output tile and
// split its K slice four ways. Each wave stages its own K tiles (global_load_lds into the same
// swizzled 128-byte rows as above) in a private STG-deep LDS ring and multiplies them, so the K
// loop waits only on the wave's own loads (no workgroup barrier) and every staged byte is read
// from LDS once (a 2 x 2 wave grid reads each A and B fragment twice). The four partial tiles are
// summed through LDS before the epilogue; the bias of each thread's epilogue columns is fetched
// before the K loop.
template <int VM>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(VM >= 0 && VM <= 63, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((VM & 15) | ((VM >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int BM, int BN, int STG, int NK, int KIND, int BMS>
__global__ __launch_bounds__(256) void gemm_wave_kernel(const bf16* __restrict__ A, int64_t lda,
                                                        const bf16* __restrict__ B, int64_t ldb, int M, int N,
                                                        int K, int splits, Epi e) {
  constexpr int NW = 4;
  constexpr int FM = BM / 16, FN = BN / 16;
  static_assert(FM * 16 == BM && FN * 16 == BN, "tile must be a multiple of 16");
  static_assert(STG == 1 || STG == 2, "ring depth");
  constexpr int ROWB = 128;
  constexpr int NBLK = (BM + BN) / 8;  // 8-row (1 KB) blocks per K tile: one load instruction each
  static_assert(NBLK * 8 == BM + BN && NBLK <= 63, "whole 8-row blocks within the vmcnt range");
  constexpr int STAGE_BYTES = (BM + BN) * ROWB;
  constexpr int WAVE_BYTES = STG * STAGE_BYTES;
  constexpr int PITCH = BN + 4;
  constexpr int RED_BYTES = NW * BM * PITCH * 4;
  constexpr int SMEM = NW * WAVE_BYTES > RED_BYTES ? NW * WAVE_BYTES : RED_BYTES;
  static_assert(SMEM <= 160 * 1024, "LDS");
  static_assert(BMS <= BM, "row step within the tile");
  constexpr int UPR = BN / 8;                      // 8-column epilogue units per row
  constexpr int UNITS = BMS * UPR;                 // the tile's first BMS rows are stored
  constexpr int UPT = (UNITS + 255) / 256;         // units per thread
  __shared__ __attribute__((aligned(1024))) char smem[SMEM];

  // the wave index read back as a scalar, so that the addresses built from it stay in SGPRs
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int Mt = (M + BMS - 1) / BMS, Nt = (N + BN - 1) / BN;
  if ((int)blockIdx.x >= Mt * Nt * splits) {  // workgroups past the tiles read e.pf ahead
    const int w = blockIdx.x - Mt * Nt * splits, nw = gridDim.x - Mt * Nt * splits;
    prefetch_part<16>(e.pf, (int64_t)w * 256 + tid, (int64_t)nw * 256);
    return;
  }
  // work id -> (split, n tile, m tile), the split outermost: an XCD's contiguous range of ids
  // covers one K slice of A rather than all of them. Up to 7 row tiles m runs fastest (the ids
  // cover all rows of a few weight slices); from 8 (576 tokens and up) in groups of 4 weight
  // slices, so that an XCD's share is a block of rows x 4 slices and its L2 fetches part of A
  // (the VAE's O: 6 x 4 tiles per XCD instead of 12 x 2)
  const int pid = xcd_remap(blockIdx.x, Mt * Nt * splits);
  int split, mt, nt;
  if (Mt >= 8) {
    grouped_tile(pid, Mt, Nt, 4, split, mt, nt);
  } else {
    split = pid / (Mt * Nt);
    const int t = pid - split * (Mt * Nt);
    nt = t / Mt;
    mt = t - nt * Mt;
  }
  const int m0 = mt * BMS, n0 = nt * BN;
  constexpr int nk = NK;                           // K tiles per wave: K = 256 NK splits (host-checked)
  const int kb = (split * NW + wave) * nk * 64;
  char* ring = smem + wave * WAVE_BYTES;

  // bias of this thread's epilogue columns (bias-less and split-K slices skip it)
  float bv[UPT][8];
  // KIND >= 0: the epilogue kind fixed at compile time (equal to e.kind); -1: read from e
  constexpr bool partial_only = KIND == OASIS_EPI_PARTIAL_F32;
  const bool has_bias = !partial_only && e.bias && e.kind != OASIS_EPI_PARTIAL_F32;
#pragma unroll
  for (int q = 0; q < UPT; ++q) {
    const int gn = min(n0 + ((tid + q * 256) % UPR) * 8, N - 8);
    f32x4 b0 = f32x4{0.f, 0.f, 0.f, 0.f}, b1 = b0;
    if (has_bias) {
      b0 = *reinterpret_cast<const f32x4*>(e.bias + gn);
      b1 = *reinterpret_cast<const f32x4*>(e.bias + gn + 4);
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      bv[q][j] = b0[j];
      bv[q][j + 4] = b1[j];
    }
  }
  // QKV + RoPE: the rotation table rows of this thread's epilogue units, fetched before the K loop
  // as well (the row's table position does not depend on the product)
  constexpr bool QKV = KIND == OASIS_EPI_QKV_ROPE;
  float rc[QKV ? UPT : 1][8], rs[QKV ? UPT : 1][8];
  if constexpr (QKV) {
#pragma unroll
    for (int q = 0; q < UPT; ++q) {
      const int u = tid + q * 256, r = u / UPR;
      const int gm = min(m0 + r, M - 1), gn = min(n0 + (u % UPR) * 8, N - 8);
      qkv_rope_tables(e, gm, gn, rc[q], rs[q]);
    }
  }

  // lane's row in each 8-row block: r = 8 blk + lane / 8, K chunk (lane % 8) ^ ((r >> 1) & 7).
  // Loads are buffer loads: a scalar base (the tile's first A row / weight row at this wave's K
  // slice), the K tile as a scalar offset and a 32-bit per-lane byte offset, below BM (BN) rows of
  // lda (ldb).
  const __amdgpu_buffer_rsrc_t Ars = buffer_rsrc(A + (int64_t)m0 * lda + kb);
  const __amdgpu_buffer_rsrc_t Brs = buffer_rsrc(B + (int64_t)n0 * ldb + kb);
  uint32_t off[NBLK];
#pragma unroll
  for (int blk = 0; blk < NBLK; ++blk) {
    const int r = blk * 8 + (lane >> 3);
    const int c = (lane & 7) ^ ((r >> 1) & 7);
    off[blk] = r < BM ? (uint32_t)(((int64_t)(min(m0 + r, M - 1) - m0) * lda + c * 8) * 2)
                      : (uint32_t)(((int64_t)(min(n0 + r - BM, N - 1) - n0) * ldb + c * 8) * 2);
  }
  auto issue = [&](int kt, int buf) {
    char* base = ring + buf * STAGE_BYTES;
#pragma unroll
    for (int blk = 0; blk < NBLK; ++blk) buffer_load_lds16(blk < BM / 8 ? Ars : Brs, off[blk], kt * 128, base + blk * 1024);
  };

  f32x4 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int lr = lane & 15, g = lane >> 4;
  auto compute = [&](int buf) {
    const char* base = ring + buf * STAGE_BYTES;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int c = ks * 4 + g;
      bf16x8 af[FM], bfr[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int r = i * 16 + lr;
        af[i] = *reinterpret_cast<const bf16x8*>(base + r * ROWB + ((c ^ ((r >> 1) & 7)) << 4));
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int r = BM + j * 16 + lr;
        bfr[j] = *reinterpret_cast<const bf16x8*>(base + r * ROWB + ((c ^ ((r >> 1) & 7)) << 4));
      }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = mfma16(af[i], bfr[j], acc[i][j]);
    }
  };

  // The scheduling barriers keep each tile's loads where they are written: the compiler would
  // otherwise sink them next to their first use and serialise the ring.
  issue(0, 0);
  if (STG == 2 && nk > 1) issue(1, 1);
#pragma unroll
  for (int k = 0; k < nk; ++k) {
    __builtin_amdgcn_sched_barrier(0);
    if (STG == 2 && k + 1 < nk)
      wait_vmcnt<NBLK>();  // tile k + 1 may still be in flight
    else
      wait_vmcnt<0>();
    __builtin_amdgcn_sched_barrier(0);
    compute(STG == 2 ? (k & 1) : 0);
    __builtin_amdgcn_sched_barrier(0);
    if (k + STG < nk) issue(k + STG, STG == 2 ? (k & 1) : 0);  // into the buffer just read
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();  // every wave is done with its ring: reuse LDS for the partial tiles

  float* red = reinterpret_cast<float*>(smem);
  float* mine = red + wave * BM * PITCH;
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) mine[(i * 16 + g * 4 + r) * PITCH + j * 16 + lr] = acc[i][j][r];
  __syncthreads();

  // thread -> (row, 8 consecutive columns): coalesced 16- / 32-byte stores
#pragma unroll
  for (int q = 0; q < UPT; ++q) {
    const int u = tid + q * 256;
    if (UNITS % 256 != 0 && u >= UNITS) break;
    const int r = u / UPR, c8 = (u % UPR) * 8;
    const int gm = m0 + r, gn = n0 + c8;
    float v[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) v[j] = bv[q][j];
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(red + w * BM * PITCH + r * PITCH + c8);
      const f32x4 c1 = *reinterpret_cast<const f32x4*>(red + w * BM * PITCH + r * PITCH + c8 + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        v[j] += c0[j];
        v[j + 4] += c1[j];
      }
    }
    if (gm < M && gn < N) {
      if (partial_only || (KIND < 0 && e.kind == OASIS_EPI_PARTIAL_F32)) {
        float* d = e.out_f32 + (int64_t)split * e.split_stride + (int64_t)gm * e.ld_out + gn;
        *reinterpret_cast<f32x4*>(d) = f32x4{v[0], v[1], v[2], v[3]};
        *reinterpret_cast<f32x4*>(d + 4) = f32x4{v[4], v[5], v[6], v[7]};
      } else if constexpr (QKV) {
        qkv_rope_store(e, gm, gn, v, rc[q], rs[q]);
      } else {
        epilogue8(e, gm, gn, v, nullptr, 0, false, KIND);
      }
    }
  }
}

// Fragment-order GEMM (at most 320 tokens): A [a_rows, K] and B [N, K] both in MFMA fragment order
// (each 16-row x 32-k block is the 64 lanes' 16-byte operands back to back), so every operand load is
// one wave reading 1 KB contiguous straight into the MFMA's registers: no LDS staging, and the whole
// K slice of a wave in flight at once. A workgroup of 8 waves owns one FM x FN block tile (16-row,
// 16-column blocks) and splits its K slice eight ways (SPW 32-wide k-steps per wave); the 8 partial
// tiles are summed through LDS (16-byte column groups XOR-swizzled by (row >> 2) & 3, which spreads
// a wave's 4-row accumulator groups over the banks), then the bias and the epilogue. Tiles are
// ordered with the split outermost, then n, then m, as in gemm_wave_kernel. Rows past M (the last
// tile's rounding) are read and their results dropped.
//
// The LayerNorm + modulate carried from O into FC1:
//  - GATED_RES_LN (O): one epilogue unit per thread, its x, gate, scale and centre fetched before
//    the MFMAs. x += gate * (acc + bias); with y = x - centre it writes y * s (fragment order), the
//    per-16-column sums of y and y^2 (the 2 threads of a 16-column group are lanes 2i, 2i + 1),
//    and, from the threads of rows m < frames, bf16 s and t of frame m as rows 2m and 2m + 1 of
//    the 16-row modulate block.
//  - GELU_TANH_LN (FC1, A = y * s) finishes it from the identity
//      (LN(x) * s + t) @ B^T = r * ((y * s) @ B^T - mu * (s @ B^T)) + t @ B^T,
//    mu and r = 1/sqrt(var + eps) being y's row mean and inverse deviation (var(y) = var(x)). The
//    modulate block is one more A block, so s @ B^T and t @ B^T of every frame come out of the same
//    MFMAs; each row's statistics are 32 lanes' loads summed by a 32-lane reduction. To leave LDS
//    for the modulate-block rows the 8 partial tiles are summed in two rounds: waves 4-7 hand
//    theirs to waves 0-3 as 16-byte lane-major stores, which add them and store the swizzled sums.
template <int FM, int FN, int SPW, int KIND>
__global__ __launch_bounds__(512) void gemm_frag_kernel(const bf16* __restrict__ A, const bf16* __restrict__ B,
                                                        int M, int N, int K, int splits, Epi e) {
  constexpr int NW = 8, TM = FM * 16, TN = FN * 16;
  constexpr bool LN = KIND == OASIS_EPI_GELU_TANH_LN;
  constexpr bool RES = KIND == OASIS_EPI_GATED_RES_LN;
  constexpr int UNITS = TM * TN / 8;
  static_assert(!RES || UNITS <= NW * 64, "GATED_RES_LN: one unit per thread");
  // LN: the modulate-block rows and row statistics beside the partial tiles; when the 8 partial
  // tiles and those do not fit in LDS together (80-row tiles), the tiles are summed in two rounds
  constexpr int LNF = LN ? NW * FN * 256 + 16 * TN + TM * 2 : 1;
  constexpr bool TWO_ROUND = LN && (NW * TM * TN + LNF) * 4 > 160 * 1024;
  constexpr int SLOTS = TWO_ROUND ? NW / 2 : NW;  // partial tiles held in LDS at once
  constexpr int ST = LN ? (TM * 32 + NW * 64 - 1) / (NW * 64) : 1;  // statistics loads per thread (at most)
  __shared__ __attribute__((aligned(16))) float red[SLOTS * TM * TN];
  __shared__ __attribute__((aligned(16))) float lnbuf[LNF];
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int Mt = (M + TM - 1) / TM, Nt = N / TN;
  if ((int)blockIdx.x >= Mt * Nt * splits) {  // workgroups past the tiles read e.pf ahead
    const int w = blockIdx.x - Mt * Nt * splits, nw = gridDim.x - Mt * Nt * splits;
    prefetch_part<8>(e.pf, (int64_t)w * (NW * 64) + tid, (int64_t)nw * (NW * 64));
    return;
  }
  const int ks = K / 32;  // k-steps per 16-row block
  const int pid = xcd_remap(blockIdx.x, Mt * Nt * splits);
  const int split = pid / (Mt * Nt);
  const int t = pid - split * (Mt * Nt);
  const int nt = t / Mt, mt = t - nt * Mt;
  const int s0 = (split * NW + wave) * SPW;  // this wave's first k-step
  const int lr = lane & 15, g = lane >> 4;
  const int vrows = LN ? 2 * ((int)fast_div((uint32_t)(M - 1), e.rpf_magic, e.rpf_shift) + 1) : 0;
  // buffer loads: the wave's first A / B block as the scalar base, 32-bit lane offsets
  const __amdgpu_buffer_rsrc_t Ars = buffer_rsrc(A + ((int64_t)mt * FM * ks + s0) * 512);
  const __amdgpu_buffer_rsrc_t Brs = buffer_rsrc(B + ((int64_t)nt * FN * ks + s0) * 512);
  i32x4 a[SPW][FM], b[SPW][FN], vb[LN ? SPW : 1];
#pragma unroll
  for (int s = 0; s < SPW; ++s) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
      a[s][i] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(Ars, ((i * ks + s) * 64 + lane) * 16, 0, 0));
#pragma unroll
    for (int j = 0; j < FN; ++j)
      b[s][j] = __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(Brs, ((j * ks + s) * 64 + lane) * 16, 0, 0));
    if constexpr (LN) {
      // only the lanes of rows 2f, 2f + 1 of the pass's frames (lane & 15 < vrows) fetch
      const __amdgpu_buffer_rsrc_t Vrs = buffer_rsrc(e.ln_mod + (int64_t)s0 * 512);
      vb[s] = lr < vrows ? __builtin_bit_cast(i32x4, __builtin_amdgcn_raw_buffer_load_b128(Vrs, (s * 64 + lane) * 16, 0, 0))
                         : i32x4{0, 0, 0, 0};
    }
  }
  // LN: this thread's piece of the tile rows' statistics (K / ln_group groups a row, two per lane:
  // 16 or 32 lanes a row)
  f32x4 st[ST];
  const int lpr_log = LN ? (e.ln_group == 32 ? 4 : 5) : 5;  // log2 of the lanes per row
  if constexpr (LN) {
    const int kg = K / e.ln_group;
#pragma unroll
    for (int q = 0; q < ST; ++q) {
      const int u = tid + q * NW * 64, r = u >> lpr_log, c = (u & ((1 << lpr_log) - 1)) * 2;
      const int gm = mt * TM + r;
      st[q] = (r < TM && gm < M && c < kg) ? *reinterpret_cast<const f32x4*>(e.ln_stats + ((int64_t)gm * kg + c) * 2)
                                          : f32x4{0.f, 0.f, 0.f, 0.f};
    }
  }
  // GATED_RES_LN: this thread's unit (row r, columns c8..c8 + 7) and its operands
  const int ur = tid / (TN / 8), uc8 = (tid - ur * (TN / 8)) * 8;
  const int um = mt * TM + ur, un = nt * TN + uc8;
  const bool unit_on = RES && tid < UNITS && um < M;
  const int ufr = RES ? (int)fast_div((uint32_t)um, e.rpf_magic, e.rpf_shift) : 0;
  const int nfr = RES ? (int)fast_div((uint32_t)(M - 1), e.rpf_magic, e.rpf_shift) + 1 : 0;
  f32x4 ux[2], ug[2], us[2], ums[2], umt[2];
  float uctr = 0.f;
  if constexpr (RES) {
    if (unit_on) {
      const float* xp = e.out_f32 + (int64_t)um * e.ld_out + un;
      const float* gp = e.gate + (int64_t)ufr * e.gate_fstride + un;
      const float* sp = e.mod_scale + (int64_t)ufr * e.gate_fstride + un;
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        ux[h] = *reinterpret_cast<const f32x4*>(xp + 4 * h);
        ug[h] = *reinterpret_cast<const f32x4*>(gp + 4 * h);
        us[h] = *reinterpret_cast<const f32x4*>(sp + 4 * h);
      }
      uctr = e.ln_center[um];
      if (um < nfr) {  // row m also carries frame m's modulate rows into the modulate block
        const float* msp = e.mod_scale + (int64_t)um * e.gate_fstride + un;
        const float* mtp = e.mod_shift + (int64_t)um * e.gate_fstride + un;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          ums[h] = *reinterpret_cast<const f32x4*>(msp + 4 * h);
          umt[h] = *reinterpret_cast<const f32x4*>(mtp + 4 * h);
        }
      }
    }
  }
  __builtin_amdgcn_sched_barrier(0);  // every load issued before the first MFMA
  f32x4 acc[FM][FN], accv[LN ? FN : 1];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int j = 0; j < (LN ? FN : 1); ++j) accv[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s = 0; s < SPW; ++s) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j)
        acc[i][j] = mfma16(__builtin_bit_cast(bf16x8, a[s][i]), __builtin_bit_cast(bf16x8, b[s][j]), acc[i][j]);
    if constexpr (LN) {
#pragma unroll
      for (int j = 0; j < FN; ++j)
        accv[j] = mfma16(__builtin_bit_cast(bf16x8, vb[s]), __builtin_bit_cast(bf16x8, b[s][j]), accv[j]);
    }
  }
  auto slot_at = [&](float* base, int i, int j, int r) -> float* {
    const int row = i * 16 + g * 4 + r, col = j * 16 + lr;
    return base + row * TN + ((((col >> 2) ^ ((row >> 2) & 3)) << 2) | (col & 3));
  };
  if constexpr (LN) {
    float* vred = lnbuf;                 // [NW][FN][64 lanes][4]: each wave's modulate-block rows
    float* vsum = vred + NW * FN * 256;  // [16][TN]
    float* rowst = vsum + 16 * TN;       // [TM] (mu, r)
    // each row's mean and 1/deviation: its lanes' (sum, sum of squares) pairs
    const float inv_k = 1.0f / (float)K;
#pragma unroll
    for (int q = 0; q < ST; ++q) {
      float sy = row16_sum(st[q][0] + st[q][2]), sq = row16_sum(st[q][1] + st[q][3]);
      if (lpr_log == 5) {
        sy = sum_xor16(sy);
        sq = sum_xor16(sq);
      }
      const int r = (tid + q * NW * 64) >> lpr_log;
      if ((lane & ((1 << lpr_log) - 1)) == 0 && r < TM) {
        const float mu = sy * inv_k;
        rowst[r * 2] = mu;
        rowst[r * 2 + 1] = rsqrtf(fmaxf(sq * inv_k - mu * mu, 0.f) + e.ln_eps);
      }
    }
    // element (row, col) of a wave's modulate-block rows sits at lane (row / 4) * 16 + col % 16,
    // register row % 4 of block col / 16; only the first vrows rows (2 per frame) are read
    auto sum_vrows = [&](int first, int stride) {
      for (int u = first; u < vrows * TN; u += stride) {
        const int row = u / TN, col = u - row * TN;
        const int off = ((col >> 4) * 64 + (row >> 2) * 16 + (col & 15)) * 4 + (row & 3);
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < NW; ++w) sum += vred[w * FN * 256 + off];
        vsum[u] = sum;
      }
    };
    if constexpr (!TWO_ROUND) {
      // every wave stores its partial tile swizzled and its modulate-block rows; then all sum the rows
      float* mine = red + wave * (TM * TN);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) *slot_at(mine, i, j, r) = acc[i][j][r];
#pragma unroll
      for (int j = 0; j < FN; ++j) *reinterpret_cast<f32x4*>(vred + ((wave * FN + j) * 64 + lane) * 4) = accv[j];
      __syncthreads();
      sum_vrows(tid, NW * 64);
      __syncthreads();
    } else {
    // round 1: waves 4-7 park their partial tiles, lane-major; every wave its modulate-block rows
    if (wave >= NW / 2) {
      float* mine = red + (wave - NW / 2) * (TM * TN);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) *reinterpret_cast<f32x4*>(mine + ((i * FN + j) * 64 + lane) * 4) = acc[i][j];
    }
#pragma unroll
    for (int j = 0; j < FN; ++j) *reinterpret_cast<f32x4*>(vred + ((wave * FN + j) * 64 + lane) * 4) = accv[j];
    __syncthreads();
    if (wave < NW / 2) {
      // round 2: waves 0-3 add the parked tile of wave + 4 (every read of it precedes this wave's
      // first write, LDS keeping a wave's operations in order) and store the sums swizzled
      float* slot = red + wave * (TM * TN);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          const f32x4 p = *reinterpret_cast<const f32x4*>(slot + ((i * FN + j) * 64 + lane) * 4);
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[i][j][r] += p[r];
        }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) *slot_at(slot, i, j, r) = acc[i][j][r];
    } else {
      sum_vrows(tid - (NW / 2) * 64, (NW / 2) * 64);  // meanwhile waves 4-7 sum the modulate-block rows
    }
    __syncthreads();
    }
    for (int u = tid; u < UNITS; u += NW * 64) {
      const int r = u / (TN / 8), c8 = (u - r * (TN / 8)) * 8;
      const int gm = mt * TM + r, gn = nt * TN + c8;
      if (gm >= M) continue;
      const int q0 = ((c8 >> 2) ^ ((r >> 2) & 3)) << 2, q1 = (((c8 >> 2) + 1) ^ ((r >> 2) & 3)) << 2;
      f32x4 a0 = f32x4{0.f, 0.f, 0.f, 0.f}, a1 = a0;
#pragma unroll
      for (int w = 0; w < SLOTS; ++w) {
        const f32x4 c0 = *reinterpret_cast<const f32x4*>(red + w * (TM * TN) + r * TN + q0);
        const f32x4 c1 = *reinterpret_cast<const f32x4*>(red + w * (TM * TN) + r * TN + q1);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
          a0[q] += c0[q];
          a1[q] += c1[q];
        }
      }
      const int fr = (int)fast_div((uint32_t)gm, e.rpf_magic, e.rpf_shift);
      const float mu = rowst[r * 2], rr = rowst[r * 2 + 1];
      const f32x4* c1p = reinterpret_cast<const f32x4*>(vsum + (2 * fr) * TN + c8);
      const f32x4* c2p = reinterpret_cast<const f32x4*>(vsum + (2 * fr + 1) * TN + c8);
      const f32x4 c10 = c1p[0], c11 = c1p[1], c20 = c2p[0], c21 = c2p[1];
      f32x4 b0 = f32x4{0.f, 0.f, 0.f, 0.f}, b1 = b0;
      if (e.bias) {
        b0 = *reinterpret_cast<const f32x4*>(e.bias + gn);
        b1 = *reinterpret_cast<const f32x4*>(e.bias + gn + 4);
      }
      float v[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        v[q] = gelu_tanh(rr * (a0[q] - mu * c10[q]) + c20[q] + b0[q]);
        v[q + 4] = gelu_tanh(rr * (a1[q] - mu * c11[q]) + c21[q] + b1[q]);
      }
      store8_bf16(e.out_bf16 + (e.out_frag ? frag_index(gm, gn, e.ld_out >> 5) : (int64_t)gm * e.ld_out + gn), v);
    }
    return;
  }
  float* mine = red + wave * (TM * TN);
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) *slot_at(mine, i, j, r) = acc[i][j][r];
  __syncthreads();
  if constexpr (RES) {
    if (tid >= UNITS || um >= M) return;  // a 16-column group's two threads leave together
    const int q0 = ((uc8 >> 2) ^ ((ur >> 2) & 3)) << 2, q1 = (((uc8 >> 2) + 1) ^ ((ur >> 2) & 3)) << 2;
    f32x4 s0v = f32x4{0.f, 0.f, 0.f, 0.f}, s1v = s0v;
    if (e.bias) {
      s0v = *reinterpret_cast<const f32x4*>(e.bias + un);
      s1v = *reinterpret_cast<const f32x4*>(e.bias + un + 4);
    }
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(red + w * (TM * TN) + ur * TN + q0);
      const f32x4 c1 = *reinterpret_cast<const f32x4*>(red + w * (TM * TN) + ur * TN + q1);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        s0v[q] += c0[q];
        s1v[q] += c1[q];
      }
    }
    float v[8], sy = 0.f, sq = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      ux[0][q] += ug[0][q] * s0v[q];
      ux[1][q] += ug[1][q] * s1v[q];
      const float y0 = ux[0][q] - uctr, y1 = ux[1][q] - uctr;
      sy += y0 + y1;
      sq += y0 * y0 + y1 * y1;
      v[q] = y0 * us[0][q];
      v[q + 4] = y1 * us[1][q];
    }
    float* xp = e.out_f32 + (int64_t)um * e.ld_out + un;
    *reinterpret_cast<f32x4*>(xp) = ux[0];
    *reinterpret_cast<f32x4*>(xp + 4) = ux[1];
    store8_bf16(e.out_bf16 + frag_index(um, un, e.ld_out >> 5), v);
    // the statistics group's threads: a pair (16 columns) on 16-column tiles, else a quad (32)
    constexpr int G = TN >= 32 ? 32 : 16;
    sy += dpp_mov<DPP_XOR1>(sy);
    sq += dpp_mov<DPP_XOR1>(sq);
    if (G == 32) {
      sy += dpp_mov<DPP_XOR2>(sy);
      sq += dpp_mov<DPP_XOR2>(sq);
    }
    if ((uc8 & (G - 1)) == 0)
      *reinterpret_cast<float2*>(e.ln_stats + ((int64_t)um * (e.ld_out / G) + un / G) * 2) = make_float2(sy, sq);
    if (um < nfr) {
      float ms[8], mt8[8];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        ms[q] = ums[0][q];
        ms[q + 4] = ums[1][q];
        mt8[q] = umt[0][q];
        mt8[q + 4] = umt[1][q];
      }
      store8_bf16(e.ln_mod + frag_index(2 * um, un, e.ld_out >> 5), ms);
      store8_bf16(e.ln_mod + frag_index(2 * um + 1, un, e.ld_out >> 5), mt8);
    }
    return;
  }
  constexpr bool partial_only = KIND == OASIS_EPI_PARTIAL_F32;
  const bool is_partial = partial_only || (KIND < 0 && e.kind == OASIS_EPI_PARTIAL_F32);
  for (int u = tid; u < UNITS; u += NW * 64) {
    const int r = u / (TN / 8), c8 = (u - r * (TN / 8)) * 8;
    const int gm = mt * TM + r, gn = nt * TN + c8;
    if (gm >= M) continue;
    f32x4 s0v = f32x4{0.f, 0.f, 0.f, 0.f}, s1v = s0v;
    if (!is_partial && e.bias) {
      s0v = *reinterpret_cast<const f32x4*>(e.bias + gn);
      s1v = *reinterpret_cast<const f32x4*>(e.bias + gn + 4);
    }
    const int q0 = ((c8 >> 2) ^ ((r >> 2) & 3)) << 2, q1 = (((c8 >> 2) + 1) ^ ((r >> 2) & 3)) << 2;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(red + w * (TM * TN) + r * TN + q0);
      const f32x4 c1 = *reinterpret_cast<const f32x4*>(red + w * (TM * TN) + r * TN + q1);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        s0v[j] += c0[j];
        s1v[j] += c1[j];
      }
    }
    if (is_partial) {
      float* d = e.out_f32 + (int64_t)split * e.split_stride + (int64_t)gm * e.ld_out + gn;
      *reinterpret_cast<f32x4*>(d) = s0v;
      *reinterpret_cast<f32x4*>(d + 4) = s1v;
    } else {
      float v[8] = {s0v[0], s0v[1], s0v[2], s0v[3], s1v[0], s1v[1], s1v[2], s1v[3]};
      epilogue8(e, gm, gn, v, nullptr, 0, false, KIND);
    }
  }
}

// the DiT's projections at one and two frames get kernels with the epilogue fixed at compile time
// (the two LN kinds exist only in these kernels: GELU_TANH_LN on tiles 4 blocks wide, GATED_RES_LN
// on 48-row tiles)
template <int FM, int FN, int SPW, int KIND>
constexpr bool frag_special() {
  if (KIND == OASIS_EPI_GELU_TANH_LN) return FN == 4;
  if (KIND == OASIS_EPI_GATED_RES_LN) return FM == 3 && FN != 3;
  return SPW == 4 && ((KIND == OASIS_EPI_QKV_ROPE && FN == 3) || (KIND == OASIS_EPI_GELU_TANH_FRAG && FN == 4) ||
                      (KIND == OASIS_EPI_PARTIAL_F32 && (FN == 4 || (FM == 3 && FN <= 2))));
}

template <int FM, int FN, int SPW, int KIND>
bool try_frag(const dim3& g, const bf16* A, const bf16* B, int M, int N, int K, int splits, const Epi& e,
              hipStream_t s) {
  if constexpr (frag_special<FM, FN, SPW, KIND>()) {
    if (e.kind == KIND) {
      hipLaunchKernelGGL((gemm_frag_kernel<FM, FN, SPW, KIND>), g, dim3(512), 0, s, A, B, M, N, K, splits, e);
      return true;
    }
  }
  return false;
}

template <int FM, int FN, int SPW>
void launch_frag3(const bf16* A, const bf16* B, int M, int N, int K, int splits, const Epi& e, hipStream_t s) {
  const int Mt = (M + FM * 16 - 1) / (FM * 16), Nt = N / (FN * 16);
  // with ranges to read ahead, workgroups past the tiles fill the CUs up to 256 (one tile each)
  const int tiles = Mt * Nt * splits;
  const dim3 g(tiles + (prefetch_any(&e.pf) && tiles < 256 ? 256 - tiles : 0));
  if (try_frag<FM, FN, SPW, OASIS_EPI_PARTIAL_F32>(g, A, B, M, N, K, splits, e, s) ||
      try_frag<FM, FN, SPW, OASIS_EPI_GELU_TANH_FRAG>(g, A, B, M, N, K, splits, e, s) ||
      try_frag<FM, FN, SPW, OASIS_EPI_QKV_ROPE>(g, A, B, M, N, K, splits, e, s) ||
      try_frag<FM, FN, SPW, OASIS_EPI_GATED_RES_LN>(g, A, B, M, N, K, splits, e, s) ||
      try_frag<FM, FN, SPW, OASIS_EPI_GELU_TANH_LN>(g, A, B, M, N, K, splits, e, s))
    return;
  hipLaunchKernelGGL((gemm_frag_kernel<FM, FN, SPW, -1>), g, dim3(512), 0, s, A, B, M, N, K, splits, e);
}

template <int FM, int FN>
void launch_frag2(int spw, const bf16* A, const bf16* B, int M, int N, int K, int splits, const Epi& e, hipStream_t s) {
  if (spw == 1) launch_frag3<FM, FN, 1>(A, B, M, N, K, splits, e, s);
  else if (spw == 2) launch_frag3<FM, FN, 2>(A, B, M, N, K, splits, e, s);
  else launch_frag3<FM, FN, 4>(A, B, M, N, K, splits, e, s);
}

// Tile of a fragment-order product, from timings of the DiT's projections at 144 and 288 tokens
// (hipGraphs of 100 launches over 32 weight copies): 80-row tiles (5 blocks) for the wide products
// over two frames (FC1, QKV and FC2's split-K slices), 48-row tiles (3 blocks) at one frame and
// for the unsplit O projection; then the widest n tile that still gives 256 workgroups (80-row
// tiles) or 192 (48-row tiles). GELU_TANH_LN tiles are 4 blocks wide, GATED_RES_LN ones 1, 2 or 4.
void frag_tile(int64_t M, int64_t N, int splits, int kind, int& fm, int& fn) {
  fm = (M <= 160 || (N <= 1024 && splits == 1)) ? 3 : 5;
  const int64_t mt = (M + fm * 16 - 1) / (fm * 16);
  const int64_t want = fm == 5 ? 256 : 192;
  fn = 0;
  if (kind == OASIS_EPI_GELU_TANH_LN) {
    fn = N % 64 == 0 ? 4 : 0;
    return;
  }
  for (int c = 4; c >= 1; --c) {
    if (kind == OASIS_EPI_GATED_RES_LN && c == 3) continue;
    if (N % (16 * c) == 0 && (fn == 0 || mt * (N / (16 * c)) * splits >= want)) {
      fn = c;
      if (mt * (N / (16 * c)) * splits >= want) break;
    }
  }
}

// The K loop is unrolled for 1, 2, 4 or 8 K tiles per wave (K / splits = 256, 512, 1024, 2048); the
// split-K, GELU and QKV + RoPE epilogues of 2 or 4 tiles per wave (the step's and the VAE's
// projections) get kernels of their own.
template <int BM, int BN, int STG, int NK, int BMS>
void launch_wave_nk(const dim3& grid, const bf16* A, int64_t lda, const bf16* B, int64_t ldb, int M, int N, int K,
                    int splits, const Epi& e, hipStream_t s) {
  const dim3 block(256);
  if (NK == 2 || NK == 4) {
    switch (e.kind) {
      case OASIS_EPI_PARTIAL_F32:
        hipLaunchKernelGGL((gemm_wave_kernel<BM, BN, STG, NK, OASIS_EPI_PARTIAL_F32, BMS>), grid, block, 0, s, A, lda, B,
                           ldb, M, N, K, splits, e);
        return;
      case OASIS_EPI_GELU_TANH:
        hipLaunchKernelGGL((gemm_wave_kernel<BM, BN, STG, NK, OASIS_EPI_GELU_TANH, BMS>), grid, block, 0, s, A, lda, B, ldb,
                           M, N, K, splits, e);
        return;
      case OASIS_EPI_GELU_TANH_FRAG:
        hipLaunchKernelGGL((gemm_wave_kernel<BM, BN, STG, NK, OASIS_EPI_GELU_TANH_FRAG, BMS>), grid, block, 0, s, A, lda, B,
                           ldb, M, N, K, splits, e);
        return;
      case OASIS_EPI_QKV_ROPE:
        hipLaunchKernelGGL((gemm_wave_kernel<BM, BN, STG, NK, OASIS_EPI_QKV_ROPE, BMS>), grid, block, 0, s, A, lda, B, ldb,
                           M, N, K, splits, e);
        return;
      default:
        break;
    }
  }
  hipLaunchKernelGGL((gemm_wave_kernel<BM, BN, STG, NK, -1, BMS>), grid, block, 0, s, A, lda, B, ldb, M, N, K, splits, e);
}

// BMS < BM: tiles start every BMS rows and compute BM (the last BM - BMS rows, which the next tile
// owns, are not stored), so that a row count such as 288 = 4 x 72 splits into whole 16-row MFMA
// blocks over more workgroups
template <int BM, int BN, int STG, int BMS = BM>
hipError_t launch_wave(const bf16* A, int64_t lda, const bf16* B, int64_t ldb, int M, int N, int K, int splits,
                       const Epi& e, hipStream_t s) {
  const int Mt = (M + BMS - 1) / BMS, Nt = (N + BN - 1) / BN;
  // with ranges to read ahead, workgroups past the tiles fill the CUs up to 256 (one tile each)
  const int tiles = Mt * Nt * splits;
  const dim3 grid(tiles + (prefetch_any(&e.pf) && tiles < 256 ? 256 - tiles : 0));
  switch ((K / splits) % 256 == 0 ? K / splits / 256 : 0) {
    case 1: launch_wave_nk<BM, BN, STG, 1, BMS>(grid, A, lda, B, ldb, M, N, K, splits, e, s); break;
    case 2: launch_wave_nk<BM, BN, STG, 2, BMS>(grid, A, lda, B, ldb, M, N, K, splits, e, s); break;
    case 4: launch_wave_nk<BM, BN, STG, 4, BMS>(grid, A, lda, B, ldb, M, N, K, splits, e, s); break;
    case 8: launch_wave_nk<BM, BN, STG, 8, BMS>(grid, A, lda, B, ldb, M, N, K, splits, e, s); break;
    default: return hipErrorInvalidConfiguration;
  }
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int STAGES, int GN = 8>
hipError_t launch_big(const bf16* A, int64_t lda, const bf16* B, int64_t ldb, int M, int N, int K, int splits,
                      const Epi& e, hipStream_t s) {
  if ((K / splits) % 64 != 0) return hipErrorInvalidConfiguration;
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  const dim3 grid(Mt * Nt * splits), block(WM * WN * 64);
  // the projections' epilogues get kernels of their own (the rest read the kind at run time)
  switch (e.kind) {
    case OASIS_EPI_QKV_ROPE:
      hipLaunchKernelGGL((gemm_big_kernel<BM, BN, WM, WN, STAGES, GN, OASIS_EPI_QKV_ROPE>), grid, block, 0, s, A, lda, B,
                         ldb, M, N, K, splits, e);
      break;
    case OASIS_EPI_GELU_TANH:
      hipLaunchKernelGGL((gemm_big_kernel<BM, BN, WM, WN, STAGES, GN, OASIS_EPI_GELU_TANH>), grid, block, 0, s, A, lda,
                         B, ldb, M, N, K, splits, e);
      break;
    case OASIS_EPI_GELU_ERF:  // the VAE's FC1
      hipLaunchKernelGGL((gemm_big_kernel<BM, BN, WM, WN, STAGES, GN, OASIS_EPI_GELU_ERF>), grid, block, 0, s, A, lda,
                         B, ldb, M, N, K, splits, e);
      break;
    case OASIS_EPI_PARTIAL_F32:
      hipLaunchKernelGGL((gemm_big_kernel<BM, BN, WM, WN, STAGES, GN, OASIS_EPI_PARTIAL_F32>), grid, block, 0, s, A,
                         lda, B, ldb, M, N, K, splits, e);
      break;
    case OASIS_EPI_GATED_RES:
      hipLaunchKernelGGL((gemm_big_kernel<BM, BN, WM, WN, STAGES, GN, OASIS_EPI_GATED_RES>), grid, block, 0, s, A, lda,
                         B, ldb, M, N, K, splits, e);
      break;
    case OASIS_EPI_RESIDUAL:
      hipLaunchKernelGGL((gemm_big_kernel<BM, BN, WM, WN, STAGES, GN, OASIS_EPI_RESIDUAL>), grid, block, 0, s, A, lda,
                         B, ldb, M, N, K, splits, e);
      break;
    default:
      hipLaunchKernelGGL((gemm_big_kernel<BM, BN, WM, WN, STAGES, GN>), grid, block, 0, s, A, lda, B, ldb, M, N, K,
                         splits, e);
  }
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int STAGES>
hipError_t launch_lds(const bf16* A, int64_t lda, const bf16* B, int64_t ldb, int M, int N, int K, int splits,
                      const Epi& e, hipStream_t s) {
  if ((K / splits) % 64 != 0) return hipErrorInvalidConfiguration;
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_lds_kernel<BM, BN, WM, WN, STAGES>), dim3(Mt * Nt * splits), dim3(256), 0, s, A, lda, B,
                     ldb, M, N, K, splits, e);
  return hipGetLastError();
}

template <int BM, int BN, int WM, int WN, int STAGES, bool BKN = false, int BKT = 64>
hipError_t launch_cfg(const bf16* A, int64_t lda, const bf16* B, int64_t ldb, int M, int N, int K,
                      int splits, const Epi& e, hipStream_t s) {
  if ((K / splits) % BKT != 0) return hipErrorInvalidConfiguration;
  const int Mt = (M + BM - 1) / BM, Nt = (N + BN - 1) / BN;
  hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, WM, WN, STAGES, BKN, BKT>), dim3(Mt * Nt * splits), dim3(256), 0, s,
                     A, lda, B, ldb, M, N, K, splits, e);
  return hipGetLastError();
}

// Tile configurations (id -> BM x BN, wave grid, prefetch depth): the ones the default choice
// below uses, for the shapes of the DiT step, the frame, the VAE and the large-token batches.
typedef hipError_t (*launch_fn)(const bf16*, int64_t, const bf16*, int64_t, int, int, int, int, const Epi&,
                                hipStream_t);
struct TileCfg {
  int bm, bn;
  launch_fn fn;
  int no_fp8_epi = 0;   // 1: its epilogue lanes do not cover aligned 32-column blocks
  int k_gran = 64;      // each split-K slice must be a multiple of this
  int k_max = 1 << 30;  // and at most this long
};
const TileCfg kTiles[] = {
    // direct-to-LDS, 4 waves: split-K slices of the O projection, QKV + RoPE at 144 / 288 tokens
    {32, 64, launch_lds<32, 64, 1, 4, 4>},                  // 0: 4 K tiles in flight
    {32, 64, launch_lds<32, 64, 1, 4, 3>},                  // 1: 3 K tiles in flight
    // the 8-wave kernel's grouped tile order and per-wave staged epilogue on 4- and 6-wave tiles:
    // FC1 / FC2 below 2048 tokens and every VAE projection
    {96, 64, launch_big<96, 64, 2, 2, 4>},                  // 2
    {64, 64, launch_big<64, 64, 2, 2, 4, 6>},               // 3: groups of 6 n tiles (576 tokens: an XCD's 54 tiles
                                                            //    are 6 whole weight slices)
    {144, 64, launch_big<144, 64, 3, 2, 4>},                // 4: 6 waves
    // 8-wave large-token tiles (2048+ tokens)
    {288, 256, launch_big<288, 256, 2, 4, 2>},              // 5
    {288, 192, launch_big<288, 192, 2, 4, 2>, 1},           // 6
    {288, 128, launch_big<288, 128, 2, 4, 2>},              // 7
    // wave-split K, 4 waves on one tile, each wave's K tiles in its own 2-deep LDS ring (K slices of
    // 256 x 1, 2, 4 or 8; not used for the fp8-block GELU epilogue)
    // 8: 80-row tiles every 72 rows: 288 tokens as 4 row blocks, so FC1 (64 weight slices) and FC2
    // (16 slices x 4 K slices) run 256 workgroups, one per CU, instead of 192 on 96-row tiles
    {72, 64, launch_wave<80, 64, 2, 72>, 1, 256, 2048},
    {48, 32, launch_wave<48, 32, 2>, 1, 256, 2048},                       // 9
    {48, 64, launch_wave<48, 64, 2>, 1, 256, 2048},                       // 10
    {64, 64, launch_wave<64, 64, 2>, 1, 256, 2048},                       // 11
    {32, 64, launch_wave<32, 64, 2>, 1, 256, 2048},                       // 12
    // large-token products of N = 1024 run unsplit (the O projection with its gated residual in
    // the epilogue): 256 workgroups at 4608 tokens, 6 waves of 48 x 64 or 8 of 144 x 16
    {144, 128, launch_big<144, 128, 3, 2, 2>},                            // 13
    {288, 64, launch_big<288, 64, 2, 4, 2>, 1},                           // 14
    {144, 128, launch_big<144, 128, 3, 2, 3>},                            // 15: 3 stages
    {144, 128, launch_big<144, 128, 3, 2, 4>},                            // 16: 4 stages
    {288, 128, launch_big<288, 128, 2, 4, 3>},                            // 17: 3 stages
};
constexpr int kNumTiles = sizeof(kTiles) / sizeof(kTiles[0]);

}  // namespace

namespace oasis {

// Default tile per shape, from timings of each projection on MI355X with cold weights (hipGraphs
// of 100 launches over rotating weight sets):
//   - 2048+ tokens: the 8-wave tall tiles, the width that fills the last round of 256 workgroups best;
//   - below, where the K slice suits the wave-split kernel (256, 512, 1024 or 2048 long):
//       FC1 (GELU): 48 x 64 (tile 10) at one 144-token frame, 80-row tiles every 72 rows x 64
//       (tile 8) up to 320 tokens (8.51 us at 288 against 9.36 on 96 x 64 tiles);
//       split-K partials of K <= 1024 (O): 48 x 32 (tile 9) up to 320 tokens, 48 x 64 (tile 10) above;
//       split-K partials of longer K (FC2): tile 10 at one frame, tile 8 up to 320 tokens;
//       other epilogues (QKV + RoPE): 32 x 64 (tile 12) at one frame, 64 x 64 (tile 11) up to 320;
//   - otherwise the shared-ring kernels: FC1 on 144 x 64 six-wave tiles (tile 4) from 512 tokens (the
//     VAE's 576) and 96 x 64 (tile 2) else; split-K partials on 32 x 64 (tile 0) for short slices up to
//     320 tokens and tile 2 else; other epilogues on 32 x 64 (tile 1), 64 x 64 (tile 3) from 512 tokens.
int auto_tile(int64_t M, int64_t N, int64_t K, int splits, int kind) {
  if (M >= 2048) return large_token_tile(M, N, kind != OASIS_EPI_GELU_TANH_FP8, 5, 6, 7);
  const int64_t Kslice = K / splits;
  const bool wave_k = Kslice % 256 == 0 && Kslice <= 2048 && ((Kslice / 256) & (Kslice / 256 - 1)) == 0;
  const bool gelu = kind == OASIS_EPI_GELU_TANH || kind == OASIS_EPI_GELU_ERF || kind == OASIS_EPI_GELU_TANH_FRAG;
  if (wave_k && M <= 320) {
    if (gelu) return M <= 160 ? 10 : 8;
    if (kind == OASIS_EPI_PARTIAL_F32) return K <= 1024 ? 9 : (M <= 160 ? 10 : 8);
    if (kind != OASIS_EPI_GELU_TANH_FP8) return M <= 160 ? 12 : 11;
  }
  if (wave_k && kind == OASIS_EPI_PARTIAL_F32 && K <= 1024) return 10;
  if (gelu) return M <= 160 ? 3 : (M >= 512 ? 4 : 2);
  if (kind == OASIS_EPI_PARTIAL_F32) {
    if (M <= 160) return Kslice <= 256 ? 0 : 2;
    return M <= 320 && Kslice <= 512 ? 0 : 2;
  }
  return M >= 512 ? 3 : 1;
}

// Split-K count for the default tile of a large-token split-K product: K slices until the
// launch has at least 256 workgroups (one per CU), within max_splits and whole 64-wide K tiles.
int gemm_auto_splits(int64_t M, int64_t N, int64_t K, int max_splits) {
  const TileCfg& t = kTiles[auto_tile(M, N, K, 1, OASIS_EPI_PARTIAL_F32)];
  const int64_t tiles = ((M + t.bm - 1) / t.bm) * ((N + t.bn - 1) / t.bn);
  int s = 1;
  while (tiles * s < 256 && 2 * s <= max_splits && 2 * s <= 8 && (K / 64) % (2 * s) == 0) s *= 2;
  return s;
}

int gemm_launch_cfg(const bf16* A, int64_t lda, const bf16* B, int64_t ldb, int64_t M, int64_t N, int64_t K,
                    const oasis_epilogue_t& ex, int tile, int splits, hipStream_t s, const Prefetch* pf) {
  OASIS_REQUIRE(A && B, OASIS_ERR_NULL, "gemm: null operand");
  OASIS_REQUIRE(aligned16(A) && aligned16(B), OASIS_ERR_ARG, "gemm: A and B must be 16-byte aligned");
  OASIS_REQUIRE(ex.kind != OASIS_EPI_GATED_RES_LN && ex.kind != OASIS_EPI_GELU_TANH_LN, OASIS_ERR_ARG,
                "gemm: epilogue kind %d runs on oasis_gemm_bf16_frag only", ex.kind);
  OASIS_REQUIRE(M > 0 && N > 0 && K > 0, OASIS_ERR_SHAPE, "gemm: empty shape M=%lld N=%lld K=%lld",
                (long long)M, (long long)N, (long long)K);
  OASIS_REQUIRE(K % BK == 0, OASIS_ERR_SHAPE, "gemm: K=%lld must be a multiple of 64", (long long)K);
  OASIS_REQUIRE(N % 8 == 0, OASIS_ERR_SHAPE, "gemm: N=%lld must be a multiple of 8", (long long)N);
  OASIS_REQUIRE(lda % 8 == 0 && ldb % 8 == 0 && lda >= K && ldb >= K, OASIS_ERR_SHAPE,
                "gemm: lda/ldb must be >= K and multiples of 8");
  OASIS_REQUIRE(M < (1ll << 31) && N < (1ll << 31), OASIS_ERR_SHAPE, "gemm: M/N too large");
  // the kernels address a tile's rows by 32-bit byte offsets from its first row
  OASIS_REQUIRE(lda < (1ll << 22) && ldb < (1ll << 22), OASIS_ERR_SHAPE, "gemm: lda/ldb must be below 2^22");
  OASIS_REQUIRE(splits >= 1 && (K / BK) % splits == 0, OASIS_ERR_SHAPE,
                "gemm: splits=%d must divide K/64=%lld", splits, (long long)(K / BK));
  Epi e = to_epi(ex);
  e.pf = prefetch_or_none(pf);
  if (const int rc = check_epilogue(e, M, N, splits)) return rc;
  if (tile < 0) tile = auto_tile(M, N, K, splits, e.kind);
  OASIS_REQUIRE(tile < kNumTiles, OASIS_ERR_ARG, "gemm: tile config %d out of range", tile);
  const TileCfg& t = kTiles[tile];
  OASIS_REQUIRE(!(t.no_fp8_epi && e.kind == OASIS_EPI_GELU_TANH_FP8), OASIS_ERR_ARG,
                "gemm: tile config %d cannot run the GELU_TANH_FP8 epilogue", tile);
  OASIS_REQUIRE((K / splits) % t.k_gran == 0 && K / splits <= t.k_max &&
                    (t.k_gran == 64 || ((K / splits / t.k_gran) & (K / splits / t.k_gran - 1)) == 0),
                OASIS_ERR_SHAPE, "gemm: tile config %d needs K/splits=%lld to be %s of %d up to %d", tile,
                (long long)(K / splits), t.k_gran == 64 ? "a multiple" : "a power-of-two multiple", t.k_gran, t.k_max);
  const hipError_t err = t.fn(A, lda, B, ldb, (int)M, (int)N, (int)K, splits, e, s);
  if (err != hipSuccess) {
    set_error("gemm launch failed: %s", hipGetErrorString(err));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

int64_t gemm_frag_rows(int64_t M) {
  const int64_t r48 = (M + 47) / 48 * 48, r80 = (M + 79) / 80 * 80;
  return M <= 160 ? r48 : std::max(r48, r80);
}

int gemm_frag_launch(const bf16* A, int64_t a_rows, const bf16* B, int64_t M, int64_t N, int64_t K,
                     const oasis_epilogue_t& ex, int splits, hipStream_t s, const Prefetch* pf) {
  OASIS_REQUIRE(A && B, OASIS_ERR_NULL, "gemm_frag: null operand");
  OASIS_REQUIRE(aligned16(A) && aligned16(B), OASIS_ERR_ARG, "gemm_frag: A and B must be 16-byte aligned");
  OASIS_REQUIRE(M > 0 && M <= 320 && M % 16 == 0, OASIS_ERR_SHAPE,
                "gemm_frag: M=%lld must be a multiple of 16 up to 320", (long long)M);
  OASIS_REQUIRE(N > 0 && N % 16 == 0 && N < (1ll << 24), OASIS_ERR_SHAPE, "gemm_frag: N=%lld must be a multiple of 16",
                (long long)N);
  OASIS_REQUIRE(splits >= 1 && K > 0 && K % splits == 0, OASIS_ERR_SHAPE, "gemm_frag: splits=%d must divide K",
                splits);
  const int64_t slice = K / splits;
  OASIS_REQUIRE(slice == 256 || slice == 512 || slice == 1024, OASIS_ERR_SHAPE,
                "gemm_frag: K/splits=%lld must be 256, 512 or 1024", (long long)slice);
  const Epi e = to_epi(ex);
  if (const int rc = check_epilogue(e, M, N, splits)) return rc;
  OASIS_REQUIRE(e.kind != OASIS_EPI_UNPATCHIFY && e.kind != OASIS_EPI_GELU_TANH_FP8, OASIS_ERR_ARG,
                "gemm_frag: epilogue kind %d is not supported", e.kind);
  int fm, fn;
  frag_tile(M, N, splits, e.kind, fm, fn);
  // the statistics' group width: GATED_RES_LN sums whole 32-column groups on tiles at least 32
  // columns wide, else 16-column ones; GELU_TANH_LN derives the same from M and its K (= O's N)
  Epi eg = e;
  eg.pf = prefetch_or_none(pf);
  if (e.kind == OASIS_EPI_GATED_RES_LN) eg.ln_group = fn >= 2 ? 32 : 16;
  if (e.kind == OASIS_EPI_GELU_TANH_LN) {
    int om, on;
    frag_tile(M, K, 1, OASIS_EPI_GATED_RES_LN, om, on);
    eg.ln_group = on >= 2 ? 32 : 16;
  }
  OASIS_REQUIRE(fn > 0, OASIS_ERR_SHAPE, "gemm_frag: N=%lld has no tile for epilogue kind %d (GELU_TANH_LN needs "
                "N %% 64 == 0)", (long long)N, e.kind);
  OASIS_REQUIRE(e.kind != OASIS_EPI_GATED_RES_LN || fm == 3, OASIS_ERR_SHAPE,
                "gemm_frag: GATED_RES_LN needs N <= 1024 and one split");
  const int64_t rows = (M + fm * 16 - 1) / (fm * 16) * (fm * 16);
  OASIS_REQUIRE(a_rows >= rows, OASIS_ERR_SHAPE, "gemm_frag: A holds %lld rows, the %d-row tiles read %lld",
                (long long)a_rows, fm * 16, (long long)rows);
  // block offsets are 32-bit byte offsets from a wave's first block
  OASIS_REQUIRE((int64_t)fm * K * 32 < (1ll << 31) && (int64_t)fn * K * 32 < (1ll << 31), OASIS_ERR_SHAPE,
                "gemm_frag: K too large");
  const int spw = (int)(slice / 256);
  const int Mi = (int)M, Ni = (int)N, Ki = (int)K;
#define OASIS_FRAG(FM_, FN_) \
  if (fm == FM_ && fn == FN_) launch_frag2<FM_, FN_>(spw, A, B, Mi, Ni, Ki, splits, eg, s)
  OASIS_FRAG(5, 4); else OASIS_FRAG(5, 3); else OASIS_FRAG(5, 2); else OASIS_FRAG(5, 1);
  else OASIS_FRAG(3, 4); else OASIS_FRAG(3, 3); else OASIS_FRAG(3, 2); else OASIS_FRAG(3, 1);
#undef OASIS_FRAG
  const hipError_t err = hipGetLastError();
  if (err != hipSuccess) {
    set_error("gemm_frag launch failed: %s", hipGetErrorString(err));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

// Default tile choice. M is small (288 / 576 tokens) and the weights are streamed once,
// so the tiles trade L2 re-reads of A and B against enough workgroups (and K-tiles in
// flight per workgroup) to keep all 256 CUs issuing HBM loads.
int gemm_launch(const bf16* A, int64_t lda, const bf16* B, int64_t ldb, int64_t M, int64_t N, int64_t K,
                const oasis_epilogue_t& ex, hipStream_t s) {
  return gemm_launch_cfg(A, lda, B, ldb, M, N, K, ex, -1, 1, s);
}

}  // namespace oasis

extern "C" int oasis_linear(const void* x, const void* w, void* out, int64_t M, int64_t K, int64_t N,
                            int w_layout, int out_dtype, oasis_stream_t stream) {
  OASIS_REQUIRE(x && w && out, OASIS_ERR_NULL, "linear: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, x, w, out), OASIS_ERR_ARG, "linear: pointers must be 16-byte aligned");
  OASIS_REQUIRE(M > 0 && N > 0 && K > 0 && K % BK == 0 && N % 8 == 0 && M < (1ll << 31) && N < (1ll << 31),
                OASIS_ERR_SHAPE, "linear: need K %% 64 == 0 and N %% 8 == 0");
  OASIS_REQUIRE(w_layout == 0 || w_layout == 1, OASIS_ERR_ARG, "linear: w_layout must be 0 ([K,N]) or 1 ([N,K])");
  OASIS_REQUIRE(out_dtype == OASIS_F32 || out_dtype == OASIS_BF16, OASIS_ERR_DTYPE, "linear: bad out dtype %d",
                out_dtype);
  oasis_epilogue_t ex;
  memset(&ex, 0, sizeof(ex));
  ex.kind = out_dtype == OASIS_F32 ? OASIS_EPI_STORE_F32 : OASIS_EPI_STORE_BF16;
  ex.out_f32 = static_cast<float*>(out);
  ex.out_bf16 = out;
  ex.ld_out = N;
  if (w_layout == 1)
    return oasis::gemm_launch(static_cast<const bf16*>(x), K, static_cast<const bf16*>(w), K, M, N, K, ex,
                              static_cast<hipStream_t>(stream));
  const Epi e = to_epi(ex);
  const hipError_t err = launch_cfg<32, 64, 1, 4, 1, true>(static_cast<const bf16*>(x), K, static_cast<const bf16*>(w),
                                                           N, (int)M, (int)N, (int)K, 1, e,
                                                           static_cast<hipStream_t>(stream));
  if (err != hipSuccess) {
    oasis::set_error("linear launch failed: %s", hipGetErrorString(err));
    return OASIS_ERR_LAUNCH;
  }
  return OASIS_OK;
}

extern "C" int oasis_gemm_bf16_config(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M,
                                      int64_t N, int64_t K, const oasis_epilogue_t* epi, int tile, int splits,
                                      oasis_stream_t stream) {
  OASIS_REQUIRE(epi, OASIS_ERR_NULL, "gemm: null epilogue");
  return oasis::gemm_launch_cfg(static_cast<const bf16*>(A), lda, static_cast<const bf16*>(B), ldb, M, N, K,
                                *epi, tile, splits, static_cast<hipStream_t>(stream));
}

extern "C" int oasis_gemm_bf16(const void* A, int64_t lda, const void* B, int64_t ldb, int64_t M,
                               int64_t N, int64_t K, const oasis_epilogue_t* epi,
                               oasis_stream_t stream) {
  OASIS_REQUIRE(epi, OASIS_ERR_NULL, "gemm: null epilogue");
  return oasis::gemm_launch(static_cast<const bf16*>(A), lda, static_cast<const bf16*>(B), ldb, M, N,
                            K, *epi, static_cast<hipStream_t>(stream));
}

extern "C" int oasis_gemm_bf16_frag(const void* A, int64_t a_rows, const void* B, int64_t M, int64_t N, int64_t K,
                                    const oasis_epilogue_t* epi, int splits, oasis_stream_t stream) {
  OASIS_REQUIRE(epi, OASIS_ERR_NULL, "gemm_frag: null epilogue");
  return oasis::gemm_frag_launch(static_cast<const bf16*>(A), a_rows, static_cast<const bf16*>(B), M, N, K, *epi,
                                 splits, static_cast<hipStream_t>(stream));
}
