// Attention kernels for gfx950.
//
// flash_kernel: flash-style multi-head attention on v_mfma_f32_16x16x32_bf16 with an
//   online softmax. A workgroup of NW waves serves one (frame, head) and NW blocks of
//   16 queries; K and V^T for 64-key chunks are staged in LDS and shared by the waves.
//   The scores are computed transposed (S^T = K Q^T) so that every lane's scores all
//   belong to one query (lane & 15): the running max/sum and the rescale of the output
//   accumulators need only lane-group reductions, and the probabilities feed the
//   P V product (as O^T = V^T P^T) straight from registers without an LDS round trip.
//   Used for spatial attention (144 tokens per frame), the VAE (576 tokens) and the
//   reference's sdpa / sdpa_causal surface (optional additive bias, causal mask).
//
// temporal_kernel: causal attention over the T frames of one (stream, position, head)
//   group. At T=2 each group is 2 queries x 2 keys, far below an MFMA tile, so it is a
//   VALU kernel: 16 lanes per group, 4 head dims per lane, dot products by 16-lane
//   butterfly reductions and an online softmax over the causal keys.
#include <type_traits>

#include "oasis_common.h"

namespace {

constexpr int KPITCH = 64 + 8;
constexpr float LOG2E = 1.4426950408889634f;

template <typename T>
__device__ __forceinline__ bf16x8 load8_bf16(const T* p);
template <>
__device__ __forceinline__ bf16x8 load8_bf16<bf16>(const bf16* p) {
  return *reinterpret_cast<const bf16x8*>(p);
}
template <>
__device__ __forceinline__ bf16x8 load8_bf16<float>(const float* p) {
  const f32x4 a = *reinterpret_cast<const f32x4*>(p);
  const f32x4 b = *reinterpret_cast<const f32x4*>(p + 4);
  float v[8] = {a[0], a[1], a[2], a[3], b[0], b[1], b[2], b[3]};
  return pack8(v);
}

// 8 consecutive K / V elements at element offset e of a (frame, head) block: bf16 blocks through a
// buffer resource (scalar base, 32-bit lane offset), which stages faster than 64-bit addresses
template <typename T>
__device__ __forceinline__ bf16x8 load8_kv(__amdgpu_buffer_rsrc_t r, const T* base, int e);
template <>
__device__ __forceinline__ bf16x8 load8_kv<bf16>(__amdgpu_buffer_rsrc_t r, const bf16*, int e) {
  return __builtin_bit_cast(bf16x8, __builtin_amdgcn_raw_buffer_load_b128(r, (uint32_t)e * 2, 0, 0));
}
template <>
__device__ __forceinline__ bf16x8 load8_kv<float>(__amdgpu_buffer_rsrc_t, const float* base, int e) {
  return load8_bf16<float>(base + e);
}

template <typename T>
__device__ __forceinline__ void store4(T* p, float a, float b, float c, float d);
template <>
__device__ __forceinline__ void store4<bf16>(bf16* p, float a, float b, float c, float d) {
  *reinterpret_cast<bf16x4*>(p) = bf16x4{f2bf(a), f2bf(b), f2bf(c), f2bf(d)};
}
template <>
__device__ __forceinline__ void store4<float>(float* p, float a, float b, float c, float d) {
  *reinterpret_cast<f32x4*>(p) = f32x4{a, b, c, d};
}

struct AttnArgs {
  int Lq, Lk;
  int64_t q_bh, kv_bh;      // element stride between (frame, head) blocks of Q and K/V
  float scale_log2;         // softmax scale * log2(e)
  const float* bias;        // [Lq, Lk] or nullptr
  int causal;
  int H;                    // heads per frame (output addressing)
  // out offset of query i, dim d of block bh: with f = bh / H, h = bh % H,
  // (f / f_inner) * o_sfo + (f % f_inner) * o_sf + h * o_sh + i * o_si + d
  int f_inner;
  int64_t o_sfo, o_sf, o_sh, o_si;
  // > 0: the output is a token-major [rows, frag_ks * 32] matrix stored in MFMA fragment order
  // (bf16): the row-major offset above names the element
  int frag_ks = 0;
  // byte ranges read by the grid slice blockIdx.z == 1 (launched when any is set)
  oasis::Prefetch pf = {{nullptr, nullptr, nullptr, nullptr}, {0, 0, 0, 0}, 7};
  // set: the output goes out as fp8 activation blocks instead (e4m3 bytes at o8 + the row-major
  // offset, the e8m0 scale of each 32-column block at o8s + offset / 32), the bf16-rounded values
  // quantized as oasis_quantize_act_fp8 would; the row-major offsets are multiples of 64 there
  uint8_t* o8 = nullptr;
  uint8_t* o8s = nullptr;
};

// Four consecutive bf16-rounded outputs r of a 32-column block whose max |v| over the block is
// amax -> e4m3 bytes (a u32) at q, and the block's e8m0 scale byte at *sc when sc is set.
__device__ __forceinline__ void store_fp8x4(uint8_t* q, uint8_t* sc, const float* r, float amax) {
  const int sb = fp8_block_scale(amax);
  const float inv = fp8_block_inv(sb);
  *reinterpret_cast<uint32_t*>(q) = pack4_fp8(r[0] * inv, r[1] * inv, r[2] * inv, r[3] * inv);
  if (sc) *sc = (uint8_t)sb;
}

// KS keys are staged in LDS at a time (K rows and V^T columns; KS >= Lk stages the whole
// sequence once, with no barrier in the key loop) and consumed in KC-key chunks.
// V^T is built from 8x8 blocks: a thread loads 8 key rows x 8 dims and transposes them in
// registers. Each V^T row (one head dim) holds its keys in k-slot order: within a 32-key
// block, position 8g + j holds the key that k-slot j of lane group g multiplies in the P V
// product (key 4g + j for j < 4, 16 + 4g + j - 4 for j >= 4), so a V fragment is one
// 16-byte LDS read. The 16-byte units of a row are XOR-swizzled by (row >> 3) & 7 within
// each 64-key group: the 8-byte staging writes of 8 dims x the same keys (rows 8 apart) and
// the fragment reads of 8 consecutive rows then fall in distinct LDS banks.
// KSPLIT = 2: two waves per 16-query block, each taking every other key chunk (two waves
// per SIMD, half the serial softmax chain each); their running (max, sum, output) states
// are merged through LDS at the end.
// PLAIN: no bias and no causal mask (only keys past Lk are masked).
template <int NW, int KC, int KS, typename T, int KSPLIT = 1, bool PLAIN = false>
__global__ __launch_bounds__(NW * KSPLIT * 64) void flash_kernel(const T* __restrict__ Q, const T* __restrict__ K,
                                                                 const T* __restrict__ V, T* __restrict__ O,
                                                                 AttnArgs a) {
  static_assert(KS % KC == 0 && KC % 32 == 0 && KS % 8 == 0, "chunking");
  static_assert(KSPLIT == 1 || KSPLIT == 2, "key split");
  static_assert(KSPLIT == 1 || KS * KPITCH * 2 >= NW * 64 * 18 * 4, "merge slots fit in the K staging");
  constexpr int VPITCH = (KS + 63) / 64 * 64 + 8;  // whole 64-key swizzle groups, +8 against bank repeats
  constexpr int KT = KC / 16;   // 16-key tiles per chunk
  constexpr int NT = NW * KSPLIT * 64;
  constexpr int KCH = KS * 8;             // 16-byte K chunks per stage
  constexpr int VBL = KS;                 // 8x8 V blocks per stage (KS/8 key blocks x 8 dim blocks)
  constexpr int KPER = (KCH + NT - 1) / NT;
  constexpr int VPER = (VBL + NT - 1) / NT;
  __shared__ __attribute__((aligned(16))) bf16 Ks[KS * KPITCH];
  __shared__ __attribute__((aligned(16))) bf16 Vt[64 * VPITCH];
  if (blockIdx.z) {  // the prefetching slice
    prefetch_lines(a.pf);
    return;
  }
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wq = wave % NW, wk = wave / NW;  // query block, key-chunk parity
  // work id -> (head, query block) with a head's query blocks on consecutive ids: xcd_remap puts
  // them on one XCD, whose L2 then fetches the head's K and V once for all of them
  const int nqb = gridDim.x;
  const int wid = xcd_remap(blockIdx.y * nqb + blockIdx.x, nqb * gridDim.y);
  const int bh = wid / nqb;
  const int q0 = ((wid - bh * nqb) * NW + wq) * 16;
  const int lr = lane & 15, g = lane >> 4;
  const T* Qb = Q + (int64_t)bh * a.q_bh;
  const T* Kb = K + (int64_t)bh * a.kv_bh;
  const T* Vb = V + (int64_t)bh * a.kv_bh;

  // this lane's query row (B operand of S^T = K Q^T): 8 dims at 8g and 32 + 8g
  const int qrow = min(q0 + lr, a.Lq - 1);
  const bf16x8 qf0 = load8_bf16<T>(Qb + (int64_t)qrow * 64 + g * 8);
  const bf16x8 qf1 = load8_bf16<T>(Qb + (int64_t)qrow * 64 + 32 + g * 8);
  const int my_q = q0 + lr;

  float m = -INFINITY, lsum = 0.f;
  f32x4 o[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) o[i] = f32x4{0.f, 0.f, 0.f, 0.f};

  const __amdgpu_buffer_rsrc_t Krs = buffer_rsrc(Kb), Vrs = buffer_rsrc(Vb);  // bf16 blocks: Lk * 128 bytes
  for (int ks0 = 0; ks0 < a.Lk; ks0 += KS) {
    __syncthreads();
    {
      bf16x8 kv[KPER], vv[VPER][8];
      // all loads of the stage first (keys past Lk read the last key; masked below)
#pragma unroll
      for (int u = 0; u < KPER; ++u) {
        const int c = min(tid + u * NT, KCH - 1);
        kv[u] = load8_kv<T>(Krs, Kb, min(ks0 + (c >> 3), a.Lk - 1) * 64 + (c & 7) * 8);
      }
#pragma unroll
      for (int u = 0; u < VPER; ++u) {
        const int b = min(tid + u * NT, VBL - 1);
        const int kb = b >> 3, db = b & 7;
#pragma unroll
        for (int r = 0; r < 8; ++r) vv[u][r] = load8_kv<T>(Vrs, Vb, min(ks0 + kb * 8 + r, a.Lk - 1) * 64 + db * 8);
      }
#pragma unroll
      for (int u = 0; u < KPER; ++u) {
        const int c = tid + u * NT;
        if (c < KCH) *reinterpret_cast<bf16x8*>(Ks + (c >> 3) * KPITCH + (c & 7) * 8) = kv[u];
      }
#pragma unroll
      for (int u = 0; u < VPER; ++u) {
        const int b = tid + u * NT;
        if (b < VBL) {
          const int kb = b >> 3, db = b & 7;
          // keys 8kb..8kb+3 go to k-slot positions p0..p0+3, keys 8kb+4..8kb+7 to p0+8..p0+11;
          // rows db*8..db*8+7 share the swizzle db
          const int p0 = (kb >> 2) * 32 + 16 * (kb & 1) + 4 * ((kb >> 1) & 1);
          const int e0 = (((p0 >> 3) ^ db) << 3) + (p0 & 7);
          const int e1 = ((((p0 >> 3) + 1) ^ db) << 3) + (p0 & 7);
#pragma unroll
          for (int j = 0; j < 8; ++j) {
            bf16* row = Vt + (db * 8 + j) * VPITCH;
            *reinterpret_cast<bf16x4*>(row + e0) = bf16x4{vv[u][0][j], vv[u][1][j], vv[u][2][j], vv[u][3][j]};
            *reinterpret_cast<bf16x4*>(row + e1) = bf16x4{vv[u][4][j], vv[u][5][j], vv[u][6][j], vv[u][7][j]};
          }
        }
      }
    }
    __syncthreads();
    if (q0 >= a.Lq) continue;

  for (int kc0 = ks0 + wk * KC; kc0 < min(ks0 + KS, a.Lk); kc0 += KC * KSPLIT) {
    const int kl = kc0 - ks0;  // chunk offset inside the staged keys
    // S^T for KT key tiles of 16: s[kt][i] = score(key kc0 + kt*16 + 4g + i, query my_q)
    float s[KT][4];
#pragma unroll
    for (int kt = 0; kt < KT; ++kt) {
      const bf16* kp = Ks + (kl + kt * 16 + lr) * KPITCH + g * 8;
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
      acc = mfma16(*reinterpret_cast<const bf16x8*>(kp), qf0, acc);
      acc = mfma16(*reinterpret_cast<const bf16x8*>(kp + 32), qf1, acc);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int key = kc0 + kt * 16 + 4 * g + i;
        float x = acc[i] * a.scale_log2;
        if (!PLAIN && a.bias && key < a.Lk && my_q < a.Lq) x += a.bias[(int64_t)my_q * a.Lk + key] * LOG2E;
        if (key >= a.Lk || (!PLAIN && a.causal && key > my_q)) x = -INFINITY;
        s[kt][i] = x;
      }
    }
    float mx = -INFINITY;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) mx = fmaxf(mx, s[kt][i]);
    mx = max_xor32(max_xor16(mx));
    const float m_new = fmaxf(m, mx);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float alpha = __builtin_amdgcn_exp2f(m - m_use);
    float ps = 0.f;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        s[kt][i] = __builtin_amdgcn_exp2f(s[kt][i] - m_use);
        ps += s[kt][i];
      }
    ps = sum_xor32(sum_xor16(ps));
    lsum = lsum * alpha + ps;
    m = m_new;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dt][i] *= alpha;

    // O^T += V^T P^T over KT/2 sub-chunks of 32 keys; k-slot j of lane group g maps to
    // key 32kc + 4g + j (j < 4) and 32kc + 16 + 4g + (j - 4) (j >= 4).
#pragma unroll
    for (int kc = 0; kc < KT / 2; ++kc) {
      bf16x8 pb;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        pb[i] = f2bf(s[2 * kc][i]);
        pb[4 + i] = f2bf(s[2 * kc + 1][i]);
      }
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const int row = dt * 16 + lr, unit = ((kl + kc * 32) >> 3) + g;
        const bf16x8 va = *reinterpret_cast<const bf16x8*>(Vt + row * VPITCH + ((unit ^ ((row >> 3) & 7)) << 3));
        o[dt] = mfma16(va, pb, o[dt]);
      }
    }
  }
  }
  if (KSPLIT > 1) {
    // lane-wise merge: both waves of a query block hold query lr's state in the same lanes
    __syncthreads();  // every wave is done with the staged K / V^T
    float* slot = reinterpret_cast<float*>(Ks) + (wq * 64 + lane) * 18;
    if (wk == 1) {
      slot[0] = m;
      slot[1] = lsum;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int i = 0; i < 4; ++i) slot[2 + dt * 4 + i] = o[dt][i];
    }
    __syncthreads();
    if (wk == 1) return;
    const float m2 = slot[0], m_new = fmaxf(m, m2);
    const float m_use = m_new == -INFINITY ? 0.f : m_new;
    const float a1 = __builtin_amdgcn_exp2f(m - m_use), a2 = __builtin_amdgcn_exp2f(m2 - m_use);
    lsum = lsum * a1 + slot[1] * a2;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) o[dt][i] = o[dt][i] * a1 + slot[2 + dt * 4 + i] * a2;
  }
  if (q0 >= a.Lq || my_q >= a.Lq) return;
  const float inv = 1.0f / lsum;
  const int f = bh / a.H, h = bh - f * a.H;
  const int fo = f / a.f_inner, fi = f - fo * a.f_inner;
  const int64_t off = fo * a.o_sfo + fi * a.o_sf + h * a.o_sh + (int64_t)my_q * a.o_si;
  const int64_t ocols = (int64_t)a.frag_ks * 32, orow = a.frag_ks ? off / ocols : 0;
  if (a.o8) {
    // dims 0..31 of the head are o[0..1] of the 4 lanes sharing lr (lane groups g), 32..63 o[2..3]
    float r[4][4], m[2] = {0.f, 0.f};
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        r[dt][i] = bf2f(f2bf(o[dt][i] * inv));
        m[dt >> 1] = fmaxf(m[dt >> 1], fabsf(r[dt][i]));
      }
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) m[h2] = max_xor32(max_xor16(m[h2]));
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int64_t e = off + dt * 16 + 4 * g;
      store_fp8x4(a.o8 + e, (g == 0 && (dt & 1) == 0) ? a.o8s + e / 32 : nullptr, r[dt], m[dt >> 1]);
    }
    return;
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const int d = dt * 16 + 4 * g;
    T* dst = a.frag_ks ? O + frag_index(orow, off - orow * ocols + d, a.frag_ks) : O + off + d;
    store4<T>(dst, o[dt][0] * inv, o[dt][1] * inv, o[dt][2] * inv, o[dt][3] * inv);
  }
}

// PLAIN variants (no bias, not causal) exist for bf16, the dtype of the DiT and VAE paths
template <int NW, int KC, int KS, typename T, int KSPLIT = 1>
void flash_go(dim3 g, const T* q, const T* k, const T* v, T* o, const AttnArgs& a, hipStream_t s) {
  const dim3 b(NW * KSPLIT * 64);
  if (oasis::prefetch_any(&a.pf)) g.z = 2;
  if constexpr (std::is_same<T, bf16>::value) {
    if (!a.bias && !a.causal) {
      hipLaunchKernelGGL((flash_kernel<NW, KC, KS, T, KSPLIT, true>), g, b, 0, s, q, k, v, o, a);
      return;
    }
  }
  hipLaunchKernelGGL((flash_kernel<NW, KC, KS, T, KSPLIT, false>), g, b, 0, s, q, k, v, o, a);
}

template <typename T>
int flash_launch(const T* q, const T* k, const T* v, T* o, int64_t n_bh, const AttnArgs& a, hipStream_t s) {
  OASIS_REQUIRE(n_bh > 0 && n_bh <= 65535, OASIS_ERR_SHAPE, "attention: bad head count %lld", (long long)n_bh);
  OASIS_REQUIRE((a.Lq / 16 + 1) * n_bh < (1ll << 31), OASIS_ERR_SHAPE, "attention: too many query blocks");
  OASIS_REQUIRE(a.Lq > 0 && a.Lk > 0, OASIS_ERR_SHAPE, "attention: empty sequence");
  // K and V rows are addressed by 32-bit offsets within a (frame, head) block
  OASIS_REQUIRE(a.Lk < (1 << 24), OASIS_ERR_SHAPE, "attention: Lk=%d must be below 2^24", a.Lk);
  // staging: short sequences (up to 32 or 64 keys: the temporal windows) and whole frames (up
  // to 160 keys, 144 per DiT frame; up to 192) in one chunk; up to 576 keys (the VAE) staged at
  // once (158 KB of LDS) and consumed in 64-key chunks by two waves per query block; longer
  // sequences in 576-key stages.
  // 144-query frames take 48 queries per workgroup (each 16-query block on two waves taking
  // alternate 32-key chunks), or with 256+ (frame, head) pairs all 144 (9 waves share one K/V
  // staging).
  const unsigned nb = (unsigned)n_bh;
  if (a.Lq <= 32 && a.Lk <= 32) {
    flash_go<2, 32, 32>(dim3(1, nb), q, k, v, o, a, s);
    return oasis::check_launch("attention");
  }
  if (a.Lq <= 64 && a.Lk <= 64) {
    flash_go<4, 64, 64>(dim3(1, nb), q, k, v, o, a, s);
    return oasis::check_launch("attention");
  }
  const int kind = a.Lk <= 160 ? 0 : (a.Lk <= 192 ? 1 : 2);
  if (a.Lq % 64 != 0 && a.Lq % 48 == 0) {
    if (kind == 0 && a.Lq % 144 == 0 && n_bh >= 256) {
      flash_go<9, 160, 160>(dim3((unsigned)(a.Lq / 144), nb), q, k, v, o, a, s);
    } else {
      const dim3 g((unsigned)(a.Lq / 48), nb);
      if (kind == 0 && n_bh <= 16)  // one frame: a workgroup per 16-query block (3x the workgroups)
        flash_go<1, 32, 160, T, 2>(dim3((unsigned)(a.Lq / 16), nb), q, k, v, o, a, s);
      else if (kind == 0)  // two waves per query block over alternate 32-key chunks
        flash_go<3, 32, 160, T, 2>(g, q, k, v, o, a, s);
      else if (kind == 1)
        flash_go<3, 192, 192>(g, q, k, v, o, a, s);
      else
        flash_go<3, 64, 576, T, 2>(g, q, k, v, o, a, s);
    }
  } else {
    const dim3 g((unsigned)((a.Lq + 63) / 64), nb);
    if (kind == 0)
      flash_go<4, 160, 160>(g, q, k, v, o, a, s);
    else if (kind == 1)
      flash_go<4, 192, 192>(g, q, k, v, o, a, s);
    else
      flash_go<4, 64, 576, T, 2>(g, q, k, v, o, a, s);
  }
  return oasis::check_launch("attention");
}

// q,k,v: [B][P][H][T][64] bf16; out: token-major [(b*T + t)*P + p][h*64 + d], row-major or
// (fks = 2H) in MFMA fragment order
__global__ __launch_bounds__(256) void temporal_kernel(const bf16* __restrict__ q, const bf16* __restrict__ k,
                                                       const bf16* __restrict__ v, bf16* __restrict__ out,
                                                       int64_t G, int T, int P, int H, float scale_log2, int qf,
                                                       int fks, oasis::Prefetch pf, uint8_t* __restrict__ out8,
                                                       uint8_t* __restrict__ out8s) {
  if (blockIdx.z) {  // the prefetching slice
    prefetch_lines(pf);
    return;
  }
  const int64_t grp = (int64_t)blockIdx.x * 16 + (threadIdx.x >> 4);
  const int j = threadIdx.x & 15;
  if (grp >= G) return;  // whole 16-lane groups exit together; no cross-group shuffles
  const int h = (int)(grp % H);
  const int64_t bp = grp / H;
  const int p = (int)(bp % P);
  const int64_t b = bp / P;
  const int64_t base = grp * T * 64 + j * 4;
  // output row `row`, this lane's 4 dims: bf16 (row-major or fragment order) or, with out8, fp8
  // blocks (the 8 lanes of an aligned 32-dim half of the head share a block)
  auto put = [&](int64_t row, float a0, float a1, float a2, float a3) {
    const int col = h * 64 + j * 4;
    if (out8) {
      const float r[4] = {bf2f(f2bf(a0)), bf2f(f2bf(a1)), bf2f(f2bf(a2)), bf2f(f2bf(a3))};
      const float amax = oct_max(fmaxf(fmaxf(fabsf(r[0]), fabsf(r[1])), fmaxf(fabsf(r[2]), fabsf(r[3]))));
      const int64_t e = row * (int64_t)(H * 64) + col;
      store_fp8x4(out8 + e, (j & 7) == 0 ? out8s + e / 32 : nullptr, r, amax);
      return;
    }
    bf16* dst = fks ? out + frag_index(row, col, fks) : out + row * (int64_t)(H * 64) + col;
    *reinterpret_cast<bf16x4*>(dst) = bf16x4{f2bf(a0), f2bf(a1), f2bf(a2), f2bf(a3)};
  };
  // qf >= 0: only query frame qf is computed, written as the single frame of a T=1 output
  // (out row b*P + p); the K/V cache path runs the current frame against cached context K/V.
  if (T == 2) {  // the DiT's 2-frame window: one round trip for all six rows
    const bf16x4 q0 = *reinterpret_cast<const bf16x4*>(q + base), q1 = *reinterpret_cast<const bf16x4*>(q + base + 64);
    const bf16x4 k0 = *reinterpret_cast<const bf16x4*>(k + base), k1 = *reinterpret_cast<const bf16x4*>(k + base + 64);
    const bf16x4 v0 = *reinterpret_cast<const bf16x4*>(v + base), v1 = *reinterpret_cast<const bf16x4*>(v + base + 64);
    // query 0 sees one causal key (softmax weight exactly 1): out_0 = v_0
    float d10 = 0.f, d11 = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      d10 += bf2f(q1[i]) * bf2f(k0[i]);
      d11 += bf2f(q1[i]) * bf2f(k1[i]);
    }
    d10 = row16_sum(d10);
    d11 = row16_sum(d11);
    (void)q0;
    const float x0 = d10 * scale_log2, x1 = d11 * scale_log2;
    const float mx = fmaxf(x0, x1);
    const float p0 = exp2f(x0 - mx), p1 = exp2f(x1 - mx);
    const float inv = 1.0f / (p0 + p1);
    const int T_out = qf < 0 ? T : 1;
    const int64_t row0 = b * T_out * P + p, row1 = qf < 0 ? row0 + P : row0;
    if (qf <= 0) put(row0, bf2f(v0[0]), bf2f(v0[1]), bf2f(v0[2]), bf2f(v0[3]));
    if (qf == 0) return;
    put(row1, (p0 * bf2f(v0[0]) + p1 * bf2f(v1[0])) * inv, (p0 * bf2f(v0[1]) + p1 * bf2f(v1[1])) * inv,
        (p0 * bf2f(v0[2]) + p1 * bf2f(v1[2])) * inv, (p0 * bf2f(v0[3]) + p1 * bf2f(v1[3])) * inv);
    return;
  }
  for (int t = qf < 0 ? 0 : qf; t < (qf < 0 ? T : qf + 1); ++t) {
    const bf16x4 qv4 = *reinterpret_cast<const bf16x4*>(q + base + t * 64);
    float qv[4] = {bf2f(qv4[0]), bf2f(qv4[1]), bf2f(qv4[2]), bf2f(qv4[3])};
    float m = -INFINITY, l = 0.f, acc[4] = {0.f, 0.f, 0.f, 0.f};
    for (int s = 0; s <= t; ++s) {
      const bf16x4 kv4 = *reinterpret_cast<const bf16x4*>(k + base + s * 64);
      float dot = qv[0] * bf2f(kv4[0]) + qv[1] * bf2f(kv4[1]) + qv[2] * bf2f(kv4[2]) + qv[3] * bf2f(kv4[3]);
      dot = row16_sum(dot);
      const float x = dot * scale_log2;
      const float m_new = fmaxf(m, x);
      const float alpha = exp2f(m - m_new);
      const float pexp = exp2f(x - m_new);
      const bf16x4 vv4 = *reinterpret_cast<const bf16x4*>(v + base + s * 64);
      l = l * alpha + pexp;
#pragma unroll
      for (int i = 0; i < 4; ++i) acc[i] = acc[i] * alpha + pexp * bf2f(vv4[i]);
      m = m_new;
    }
    const float inv = 1.0f / l;
    const int64_t frame = qf < 0 ? b * T + t : b;
    put(frame * P + p, acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
  }
}

}  // namespace

namespace {

int attention_impl(const void* q, const void* k, const void* v, void* out, int64_t n_frames, int64_t L,
                   int64_t n_heads, float scale, hipStream_t stream, bool out_frag,
                   const oasis::Prefetch* pf = nullptr, uint8_t* out8 = nullptr, uint8_t* out8_scale = nullptr) {
  OASIS_REQUIRE(q && k && v && out, OASIS_ERR_NULL, "attention: null pointer");
  OASIS_REQUIRE(!out8 || (out8_scale && !out_frag), OASIS_ERR_ARG,
                "attention: an fp8 output needs its scales and a row-major layout");
  OASIS_REQUIRE(!out_frag || (n_frames * L) % 16 == 0, OASIS_ERR_SHAPE,
                "attention: a fragment-order output needs a multiple of 16 rows");
  OASIS_REQUIRE(oasis_aligned(16, q, k, v, out), OASIS_ERR_ARG, "attention: pointers must be 16-byte aligned");
  OASIS_REQUIRE(n_frames > 0 && L > 0 && n_heads > 0 && L < (1 << 30), OASIS_ERR_SHAPE, "attention: bad shape");
  AttnArgs a;
  a.Lq = a.Lk = (int)L;
  a.q_bh = a.kv_bh = L * 64;
  a.scale_log2 = scale * LOG2E;
  a.bias = nullptr;
  a.causal = 0;
  a.H = (int)n_heads;
  a.f_inner = 1 << 30;
  a.o_sfo = 0;
  a.o_sf = L * n_heads * 64;
  a.o_sh = 64;
  a.o_si = n_heads * 64;
  a.frag_ks = out_frag ? (int)(n_heads * 2) : 0;
  a.pf = oasis::prefetch_or_none(pf);
  a.o8 = out8;
  a.o8s = out8_scale;
  return flash_launch<bf16>(static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v),
                            static_cast<bf16*>(out), n_frames * n_heads, a, stream);
}

}  // namespace

extern "C" int oasis_attention(const void* q, const void* k, const void* v, void* out, int64_t n_frames, int64_t L,
                               int64_t n_heads, float scale, oasis_stream_t stream) {
  return attention_impl(q, k, v, out, n_frames, L, n_heads, scale, static_cast<hipStream_t>(stream), false);
}

extern "C" int oasis_sdpa(const void* Q, const void* K, const void* V, void* out, int64_t n_heads_total, int64_t sq,
                          int64_t skv, int64_t head_dim, float scale, const float* bias, int causal, int dtype,
                          oasis_stream_t stream) {
  OASIS_REQUIRE(Q && K && V && out, OASIS_ERR_NULL, "sdpa: null pointer");
  OASIS_REQUIRE(oasis_aligned(16, Q, K, V, out), OASIS_ERR_ARG, "sdpa: pointers must be 16-byte aligned");
  OASIS_REQUIRE(head_dim == 64, OASIS_ERR_SHAPE, "sdpa: head_dim must be 64");
  OASIS_REQUIRE(sq > 0 && skv > 0 && sq < (1 << 30) && skv < (1 << 30), OASIS_ERR_SHAPE, "sdpa: bad shape");
  AttnArgs a;
  a.Lq = (int)sq;
  a.Lk = (int)skv;
  a.q_bh = sq * 64;
  a.kv_bh = skv * 64;
  a.scale_log2 = scale * LOG2E;
  a.bias = bias;
  a.causal = causal;
  a.H = 1;
  a.f_inner = 1 << 30;
  a.o_sfo = 0;
  a.o_sf = sq * 64;
  a.o_sh = 0;
  a.o_si = 64;
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (dtype == OASIS_BF16)
    return flash_launch<bf16>(static_cast<const bf16*>(Q), static_cast<const bf16*>(K), static_cast<const bf16*>(V),
                              static_cast<bf16*>(out), n_heads_total, a, s);
  if (dtype == OASIS_F32)
    return flash_launch<float>(static_cast<const float*>(Q), static_cast<const float*>(K),
                               static_cast<const float*>(V), static_cast<float*>(out), n_heads_total, a, s);
  oasis::set_error("sdpa: unsupported dtype %d", dtype);
  return OASIS_ERR_DTYPE;
}

namespace oasis {

int attention(const void* q, const void* k, const void* v, void* out, int64_t n_frames, int64_t L, int64_t n_heads,
              float scale, hipStream_t stream, bool out_frag, const Prefetch* pf, uint8_t* out8, uint8_t* out8_scale) {
  return attention_impl(q, k, v, out, n_frames, L, n_heads, scale, stream, out_frag, pf, out8, out8_scale);
}

int attention_frag(const void* q, const void* k, const void* v, void* out, int64_t n_frames, int64_t L,
                   int64_t n_heads, float scale, hipStream_t stream) {
  return attention_impl(q, k, v, out, n_frames, L, n_heads, scale, stream, true);
}

int temporal_attention(const void* q, const void* k, const void* v, void* out, int64_t B, int64_t T, int64_t P,
                       int64_t n_heads, float scale, int q_frame, hipStream_t stream, bool out_frag,
                       const Prefetch* pf, uint8_t* out8, uint8_t* out8_scale) {
  OASIS_REQUIRE(q && k && v && out, OASIS_ERR_NULL, "temporal_attention: null pointer");
  OASIS_REQUIRE(!out8 || (out8_scale && !out_frag), OASIS_ERR_ARG,
                "temporal_attention: an fp8 output needs its scales and a row-major layout");
  OASIS_REQUIRE(!out_frag || (B * (q_frame < 0 ? T : 1) * P) % 16 == 0, OASIS_ERR_SHAPE,
                "temporal_attention: a fragment-order output needs a multiple of 16 rows");
  OASIS_REQUIRE(oasis_aligned(16, q, k, v, out), OASIS_ERR_ARG, "temporal_attention: pointers must be 16-byte aligned");
  OASIS_REQUIRE(B > 0 && T > 0 && P > 0 && n_heads > 0 && T <= 4096, OASIS_ERR_SHAPE,
                "temporal_attention: bad shape");
  OASIS_REQUIRE(q_frame < T, OASIS_ERR_ARG, "temporal_attention: q_frame must be < T");
  const int64_t G = B * P * n_heads;
  if (T >= 8 && q_frame < 0) {
    // long causal windows on the MFMA flash kernel: each (stream, position, head) group is a
    // contiguous [T][64] block; outputs land token-major at row (b*T + t)*P + p
    OASIS_REQUIRE(G <= 65535, OASIS_ERR_SHAPE, "temporal_attention: too many (stream, position, head) groups");
    AttnArgs a;
    a.Lq = a.Lk = (int)T;
    a.q_bh = a.kv_bh = T * 64;
    a.scale_log2 = scale * LOG2E;
    a.bias = nullptr;
    a.causal = 1;
    a.H = (int)n_heads;
    a.f_inner = (int)P;  // f = b*P + p
    a.o_sfo = T * P * n_heads * 64;
    a.o_sf = n_heads * 64;
    a.o_sh = 64;
    a.o_si = P * n_heads * 64;
    a.frag_ks = out_frag ? (int)(n_heads * 2) : 0;
    a.pf = prefetch_or_none(pf);
    a.o8 = out8;
    a.o8s = out8_scale;
    return flash_launch<bf16>(static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v),
                              static_cast<bf16*>(out), G, a, stream);
  }
  hipLaunchKernelGGL(temporal_kernel, dim3((unsigned)((G + 15) / 16), 1, prefetch_any(pf) ? 2 : 1), dim3(256), 0,
                     stream, static_cast<const bf16*>(q), static_cast<const bf16*>(k), static_cast<const bf16*>(v),
                     static_cast<bf16*>(out), G, (int)T, (int)P, (int)n_heads, scale * LOG2E, q_frame < 0 ? -1 : q_frame,
                     out_frag ? (int)(n_heads * 2) : 0, prefetch_or_none(pf), out8, out8_scale);
  return check_launch("temporal_attention");
}

}  // namespace oasis

extern "C" int oasis_temporal_attention(const void* q, const void* k, const void* v, void* out, int64_t B, int64_t T,
                                        int64_t P, int64_t n_heads, float scale, oasis_stream_t stream) {
  return oasis::temporal_attention(q, k, v, out, B, T, P, n_heads, scale, -1, static_cast<hipStream_t>(stream));
}

extern "C" int oasis_attention_fp8(const void* q, const void* k, const void* v, void* out8, void* out8_scale,
                                   int64_t n_frames, int64_t L, int64_t n_heads, float scale, oasis_stream_t stream) {
  OASIS_REQUIRE(out8 && out8_scale, OASIS_ERR_NULL, "attention_fp8: null output");
  return attention_impl(q, k, v, out8, n_frames, L, n_heads, scale, static_cast<hipStream_t>(stream), false, nullptr,
                        static_cast<uint8_t*>(out8), static_cast<uint8_t*>(out8_scale));
}

extern "C" int oasis_temporal_attention_fp8(const void* q, const void* k, const void* v, void* out8, void* out8_scale,
                                            int64_t B, int64_t T, int64_t P, int64_t n_heads, float scale,
                                            oasis_stream_t stream) {
  OASIS_REQUIRE(out8 && out8_scale, OASIS_ERR_NULL, "temporal_attention_fp8: null output");
  return oasis::temporal_attention(q, k, v, out8, B, T, P, n_heads, scale, -1, static_cast<hipStream_t>(stream), false,
                                   nullptr, static_cast<uint8_t*>(out8), static_cast<uint8_t*>(out8_scale));
}
