// Epilogue of the projection GEMMs (bf16 and fp8 kernels share it): the device-side
// copy of oasis_epilogue_t, the XCD-aware workgroup order and the 8-column epilogue.
#pragma once

#include "oasis_common.h"

namespace {



// pitch (floats) of a position's row in the LDS copy of the QKV rotation tables (rope_to_lds)
constexpr int ROPE_TP = 68;

struct Epi {
  int kind;
  int n_heads;
  const float* bias;
  float* out_f32;
  bf16* out_bf16;
  int64_t ld_out;
  const float* gate;
  int64_t gate_fstride;
  int64_t rows_per_frame;
  int64_t frames_per_stream;
  bf16* q;
  bf16* k;
  bf16* v;
  const float* rope_cos;
  const float* rope_sinp;
  int rope_by_frame;
  int unpatch_grid_w;
  int64_t s_b, s_t, s_p, s_h;
  int unpatch_patch;
  int unpatch_channels;
  int64_t split_stride;
  uint8_t* out_fp8;
  uint8_t* out_scale;
  int64_t ld_scale;
  const float* mod_scale;
  const float* mod_shift;
  const float* ln_center;
  float* ln_stats;
  bf16* ln_mod;
  float ln_eps;
  int out_frag;
  int ln_group;  // *_LN: columns per statistics group (16 or 32), set by the fragment-order launcher
  oasis::Prefetch pf;  // ranges read ahead by the workgroups past the tiles (wave-split, fragment order)
  // n / rows_per_frame and n / frames_per_stream as (n * magic) >> shift (see DivMagic)
  uint64_t rpf_magic, fps_magic;
  int rpf_shift, fps_shift;
};

// Exact unsigned division by a fixed d >= 1 for any n < 2^31: magic = ceil(2^s / d) with
// s = 32 + ceil(log2 d), so magic < 2^33, n * magic < 2^64, and the error n (magic - 2^s/d) / 2^s
// stays below 1/d, which cannot carry floor(n/d) to the next integer.
struct DivMagic {
  uint64_t magic;
  int shift;
};
inline DivMagic div_magic(uint64_t d) {
  if (d == 0 || d >= (1ull << 31)) return DivMagic{0, 0};  // unused: the host checks reject such shapes
  int l = 0;
  while ((1ull << l) < d) ++l;
  const int s = 32 + l;
  const unsigned __int128 one = 1;
  return DivMagic{(uint64_t)(((one << s) + d - 1) / d), s};
}
__device__ __forceinline__ uint32_t fast_div(uint32_t n, uint64_t magic, int shift) {
  return (uint32_t)(((uint64_t)n * magic) >> shift);
}


// Large-token tile order: pid -> (split, m tile, n tile) with the split outermost, then groups
// of GN n tiles in which n runs fastest, so consecutive ids (one XCD's share after xcd_remap)
// cover a compact (count / GN) x GN block of tiles.
__device__ __forceinline__ void grouped_tile(int pid, int Mt, int Nt, int GN, int& split, int& mt, int& nt) {
  const int per = Mt * Nt;
  split = pid / per;
  const int t = pid - split * per;
  const int in_group = GN * Mt;
  const int grp = t / in_group, first = grp * GN;
  const int gsz = min(Nt - first, GN);
  const int r = t - grp * in_group;
  mt = r / gsz;
  nt = first + (r - mt * gsz);
}

// Large-token tile choice among 288 x 256, 288 x 192 (only when allow192) and 288 x 128 (ids
// t256, t192, t128): among the widths that divide N, the one whose tile count fills its last
// round of 256 workgroups best (ties: the wider tile); 288 x 128 when none divides N.
inline int large_token_tile(int64_t M, int64_t N, bool allow192, int t256, int t192, int t128) {
  const int64_t mt = (M + 287) / 288;
  const int widths[3] = {256, 192, 128};
  const int ids[3] = {t256, t192, t128};
  int best = t128;
  double best_fill = -1.0;
  for (int i = 0; i < 3; ++i) {
    if (N % widths[i] != 0 || (widths[i] == 192 && !allow192)) continue;
    const int64_t tiles = mt * (N / widths[i]);
    const int64_t rounds = (tiles + 255) / 256;
    const double fill = (double)tiles / (double)(rounds * 256);
    if (fill > best_fill + 1e-9) {
      best_fill = fill;
      best = ids[i];
    }
  }
  return best;
}

// 16 (or 4) bytes per lane from global memory straight into LDS at lds + 16 * lane (4 * lane);
// lds is wave-uniform.
__device__ __forceinline__ void load_lds16(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, reinterpret_cast<uint32_t*>(lds), 16, 0, 0);
}
__device__ __forceinline__ void load_lds4(const void* g, void* lds) {
  __builtin_amdgcn_global_load_lds(g, reinterpret_cast<uint32_t*>(lds), 4, 0, 0);
}

// The same from a buffer (buffer_rsrc): a 32-bit per-lane byte offset voff and a scalar byte
// offset soff.
__device__ __forceinline__ void buffer_load_lds16(__amdgpu_buffer_rsrc_t rsrc, uint32_t voff, uint32_t soff, void* lds) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}

__device__ __forceinline__ void store8_bf16(bf16* dst, const float* v) {
  *reinterpret_cast<bf16x8*>(dst) = pack8(v);
}

// QKV_ROPE in two parts, so a caller can fetch the rotation tables of its next rows while it
// finishes the current ones: the cos / signed-sin entries of (row m, columns n0..n0+7) (only
// q and k columns are rotated), then the rotation, head split and store.
// tab (optional): an LDS copy of the tables, tab_rows cos rows of 64 then tab_rows sin rows.
__device__ __forceinline__ void qkv_rope_tables(const Epi& e, int64_t m, int n0, float* c, float* sn,
                                                const float* tab = nullptr, int tab_rows = 0) {
  const int D = e.n_heads * 64;
  const int which = (n0 >= D) + (n0 >= 2 * D);  // 0 q, 1 k, 2 v
  if (which == 2) return;
  const int d0 = (n0 - which * D) & 63;
  // 32-bit index math (M, rows and frames are < 2^31; checked on the host)
  const uint32_t rpf = (uint32_t)e.rows_per_frame, fps = (uint32_t)e.frames_per_stream;
  const uint32_t f = fast_div((uint32_t)m, e.rpf_magic, e.rpf_shift), p = (uint32_t)m - f * rpf;
  const uint32_t t = f - fast_div(f, e.fps_magic, e.fps_shift) * fps;
  const uint32_t pos = e.rope_by_frame ? t : p;
  const float* cp = tab ? tab + pos * ROPE_TP + d0 : e.rope_cos + pos * 64 + d0;
  const float* sp = tab ? tab + (tab_rows + pos) * ROPE_TP + d0 : e.rope_sinp + pos * 64 + d0;
  const f32x4 c0 = *reinterpret_cast<const f32x4*>(cp);
  const f32x4 c1 = *reinterpret_cast<const f32x4*>(cp + 4);
  const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp);
  const f32x4 s1 = *reinterpret_cast<const f32x4*>(sp + 4);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    c[j] = c0[j];
    c[j + 4] = c1[j];
    sn[j] = s0[j];
    sn[j + 4] = s1[j];
  }
}

// The rotation of 8 consecutive values: v[j] = v[j] c[j] + v[j ^ 1] s[j], one fused multiply-add
// each, written out so that every QKV epilogue rounds alike
__device__ __forceinline__ void rope_rotate8(float* v, const float* c, const float* sn) {
  float r[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) r[j] = __builtin_fmaf(v[j], c[j], v[j ^ 1] * sn[j]);
#pragma unroll
  for (int j = 0; j < 8; ++j) v[j] = r[j];
}

__device__ __forceinline__ void qkv_rope_store(const Epi& e, int64_t m, int n0, float* v, const float* c,
                                               const float* sn) {
  const int D = e.n_heads * 64;
  const int which = (n0 >= D) + (n0 >= 2 * D);
  const int nn = n0 - which * D;
  const int h = nn >> 6, d0 = nn & 63;
  const uint32_t rpf = (uint32_t)e.rows_per_frame, fps = (uint32_t)e.frames_per_stream;
  const uint32_t f = fast_div((uint32_t)m, e.rpf_magic, e.rpf_shift), p = (uint32_t)m - f * rpf;
  const uint32_t b = fast_div(f, e.fps_magic, e.fps_shift), t = f - b * fps;
  if (which < 2) rope_rotate8(v, c, sn);
  bf16* base = which == 0 ? e.q : (which == 1 ? e.k : e.v);
  store8_bf16(base + (int64_t)b * e.s_b + (int64_t)t * e.s_t + (int64_t)p * e.s_p + (int64_t)h * e.s_h + d0, v);
}

// QKV + RoPE + head split in the large-token kernels' per-wave epilogue, where lane l takes the 8
// columns ((l + 64 q) % upr) * 8 of row (l + 64 q) / upr of every 16-row group in pass q. What a
// lane's columns decide (q, k or v; head; dimension; rotated or not) is worked out once per pass,
// each 16-row group steps the row through position, frame and stream, and stores go through
// 32-bit offsets (check_epilogue keeps every q / k / v offset below 2^31).
template <int NPASS>
struct QkvRows {
  bf16* base[NPASS];
  int col[NPASS], d0[NPASS];
  bool rot[NPASS];
  uint32_t p[NPASS], t[NPASS], s[NPASS];  // pass q's row in the current group: position, frame, stream

  // n_first: the wave's first column; m_first: its first row
  __device__ __forceinline__ void init(const Epi& e, int lane, int upr, int n_first, int m_first) {
    const int D = e.n_heads * 64;
#pragma unroll
    for (int q = 0; q < NPASS; ++q) {
      const int gn = n_first + ((lane + 64 * q) % upr) * 8;
      const int which = (gn >= D) + (gn >= 2 * D);
      const int nn = gn - which * D;
      base[q] = which == 0 ? e.q : (which == 1 ? e.k : e.v);
      d0[q] = nn & 63;
      col[q] = (nn >> 6) * (int)e.s_h + d0[q];
      rot[q] = which < 2;
      const uint32_t gm = (uint32_t)(m_first + (lane + 64 * q) / upr);
      const uint32_t f = fast_div(gm, e.rpf_magic, e.rpf_shift);
      p[q] = gm - f * (uint32_t)e.rows_per_frame;
      s[q] = fast_div(f, e.fps_magic, e.fps_shift);
      t[q] = f - s[q] * (uint32_t)e.frames_per_stream;
    }
  }
  // a[q] by unrolled selects: q is only known at run time, and indexing the arrays with it would
  // put them in scratch memory
  template <typename T>
  static __device__ __forceinline__ T pick(const T (&a)[NPASS], int q) {
    T r = a[0];
#pragma unroll
    for (int i = 1; i < NPASS; ++i)
      if (q == i) r = a[i];
    return r;
  }
  // rotate (q and k) and store 8 values of pass q's row; tab / tab_rows: the LDS copy of the tables
  __device__ __forceinline__ void store(const Epi& e, int q, float* v, const float* tab, int tab_rows) const {
    const uint32_t pq = pick(p, q), tq = pick(t, q), sq = pick(s, q);
    const int dq = pick(d0, q);
    if (pick(rot, q)) {
      const uint32_t pos = e.rope_by_frame ? tq : pq;
      const float* cp = tab_rows ? tab + pos * ROPE_TP + dq : e.rope_cos + pos * 64 + dq;
      const float* sp = tab_rows ? tab + (tab_rows + pos) * ROPE_TP + dq : e.rope_sinp + pos * 64 + dq;
      const f32x4 c0 = *reinterpret_cast<const f32x4*>(cp), c1 = *reinterpret_cast<const f32x4*>(cp + 4);
      const f32x4 s0 = *reinterpret_cast<const f32x4*>(sp), s1 = *reinterpret_cast<const f32x4*>(sp + 4);
      const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
      const float sn[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
      rope_rotate8(v, c, sn);
    }
    const uint32_t off = sq * (uint32_t)e.s_b + tq * (uint32_t)e.s_t + pq * (uint32_t)e.s_p + (uint32_t)pick(col, q);
    store8_bf16(pick(base, q) + off, v);
  }
  // on to the next 16-row group
  __device__ __forceinline__ void advance(const Epi& e) {
    const uint32_t rpf = (uint32_t)e.rows_per_frame, fps = (uint32_t)e.frames_per_stream;
#pragma unroll
    for (int q = 0; q < NPASS; ++q) {
      p[q] += 16;
      while (p[q] >= rpf) {
        p[q] -= rpf;
        if (++t[q] == fps) {
          t[q] = 0;
          ++s[q];
        }
      }
    }
  }
};

// The residual epilogues (GATED_RES, RESIDUAL) in the large-token kernels' per-wave epilogue, with
// the lane-to-unit map of QkvRows: the x (and gate) vectors of a 16-row group are fetched one group
// ahead, into buffer b = group & 1, so that only the first group's memory round trip is exposed.
// No other lane or workgroup writes the x elements a lane fetches.
template <int UPR, int KIND>
struct ResAhead {
  static_assert(KIND == OASIS_EPI_GATED_RES || KIND == OASIS_EPI_RESIDUAL, "residual kinds");
  static constexpr int UPL = (16 * UPR + 63) / 64;
  f32x4 x[2][UPL][2], g[2][UPL][2];

  // the unit of pass q: its row within the group and its first column within the wave's tile
  static __device__ __forceinline__ int row(int lane, int q) { return (lane + 64 * q) / UPR; }
  static __device__ __forceinline__ int col(int lane, int q) { return ((lane + 64 * q) % UPR) * 8; }
  static __device__ __forceinline__ bool live(int lane, int q) { return lane + 64 * q < 16 * UPR; }

  // row0 / col0: the group's first row and the wave's first column
  __device__ __forceinline__ void fetch(const Epi& e, int lane, int row0, int col0, int M, int N, int b) {
#pragma unroll
    for (int q = 0; q < UPL; ++q) {
      const int gm = row0 + row(lane, q), gn = col0 + col(lane, q);
      if (!live(lane, q) || gm >= M || gn >= N) continue;
      const float* d = e.out_f32 + (int64_t)gm * e.ld_out + gn;
      x[b][q][0] = *reinterpret_cast<const f32x4*>(d);
      x[b][q][1] = *reinterpret_cast<const f32x4*>(d + 4);
      if constexpr (KIND == OASIS_EPI_GATED_RES) {
        const int64_t f = fast_div((uint32_t)gm, e.rpf_magic, e.rpf_shift);
        const float* gp = e.gate + f * e.gate_fstride + gn;
        g[b][q][0] = *reinterpret_cast<const f32x4*>(gp);
        g[b][q][1] = *reinterpret_cast<const f32x4*>(gp + 4);
      }
    }
  }
  // x[gm, gn .. gn + 8) += (gate *) v with the vectors fetched for pass q into buffer b
  __device__ __forceinline__ void store(const Epi& e, int q, int b, int64_t gm, int gn, const float* v) const {
    f32x4 x0 = x[b][q][0], x1 = x[b][q][1];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      if constexpr (KIND == OASIS_EPI_GATED_RES) {
        x0[j] += g[b][q][0][j] * v[j];
        x1[j] += g[b][q][1][j] * v[j + 4];
      } else {
        x0[j] += v[j];
        x1[j] += v[j + 4];
      }
    }
    float* d = e.out_f32 + gm * e.ld_out + gn;
    *reinterpret_cast<f32x4*>(d) = x0;
    *reinterpret_cast<f32x4*>(d + 4) = x1;
  }
};

// Applies the epilogue to 8 consecutive columns [n0, n0+8) of row m (all < N). tab / tab_rows:
// an LDS copy of the QKV rotation tables (see rope_lds_rows), or null. with_bias = false: the
// caller has already added the bias. kind >= 0: the epilogue kind known at compile time (it must
// equal e.kind), which drops the other kinds' code.
__device__ __forceinline__ void epilogue8(const Epi& e, int64_t m, int n0, float* v, const float* tab = nullptr,
                                          int tab_rows = 0, bool with_bias = true, int kind = -1) {
  if (with_bias && e.bias) {
    const f32x4 b0 = *reinterpret_cast<const f32x4*>(e.bias + n0);
    const f32x4 b1 = *reinterpret_cast<const f32x4*>(e.bias + n0 + 4);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      v[j] += b0[j];
      v[j + 4] += b1[j];
    }
  }
  switch (kind >= 0 ? kind : e.kind) {
    case OASIS_EPI_STORE_F32: {
      float* d = e.out_f32 + m * e.ld_out + n0;
      *reinterpret_cast<f32x4*>(d) = f32x4{v[0], v[1], v[2], v[3]};
      *reinterpret_cast<f32x4*>(d + 4) = f32x4{v[4], v[5], v[6], v[7]};
      break;
    }
    case OASIS_EPI_STORE_BF16:
      store8_bf16(e.out_bf16 + m * e.ld_out + n0, v);
      break;
    case OASIS_EPI_GELU_TANH: {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = gelu_tanh(v[j]);
      store8_bf16(e.out_bf16 + m * e.ld_out + n0, v);
      break;
    }
    case OASIS_EPI_GELU_ERF: {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = gelu_erf(v[j]);
      store8_bf16(e.out_bf16 + m * e.ld_out + n0, v);
      break;
    }
    case OASIS_EPI_GATED_RES: {
      const int64_t f = fast_div((uint32_t)m, e.rpf_magic, e.rpf_shift);
      const float* g = e.gate + f * e.gate_fstride + n0;
      float* d = e.out_f32 + m * e.ld_out + n0;
      f32x4 x0 = *reinterpret_cast<f32x4*>(d), x1 = *reinterpret_cast<f32x4*>(d + 4);
      const f32x4 g0 = *reinterpret_cast<const f32x4*>(g), g1 = *reinterpret_cast<const f32x4*>(g + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x0[j] += g0[j] * v[j];
        x1[j] += g1[j] * v[j + 4];
      }
      *reinterpret_cast<f32x4*>(d) = x0;
      *reinterpret_cast<f32x4*>(d + 4) = x1;
      break;
    }
    case OASIS_EPI_RESIDUAL: {
      float* d = e.out_f32 + m * e.ld_out + n0;
      f32x4 x0 = *reinterpret_cast<f32x4*>(d), x1 = *reinterpret_cast<f32x4*>(d + 4);
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        x0[j] += v[j];
        x1[j] += v[j + 4];
      }
      *reinterpret_cast<f32x4*>(d) = x0;
      *reinterpret_cast<f32x4*>(d + 4) = x1;
      break;
    }
    case OASIS_EPI_QKV_ROPE: {
      float c[8], sn[8];
      qkv_rope_tables(e, m, n0, c, sn, tab, tab_rows);
      qkv_rope_store(e, m, n0, v, c, sn);
      break;
    }
    case OASIS_EPI_UNPATCHIFY: {
      // m = f*gh*gw + hh*gw + ww; n = (c*ps + pp)*ps + qq -> frame f [c][hh*ps + pp][ww*ps + qq]
      const int ps = e.unpatch_patch, gw = e.unpatch_grid_w;
      const int64_t f = m / e.rows_per_frame, mm = m - f * e.rows_per_frame;
      const int64_t hh = mm / gw, ww = mm - hh * gw;
      const int64_t W = (int64_t)gw * ps;
      const int64_t H = e.rows_per_frame / gw * ps;  // rows_per_frame = gh*gw
      float* out = e.out_f32 + f * 3 * H * W;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int n = n0 + j;
        const int c = n / (ps * ps), rem = n - c * ps * ps;
        const int pp = rem / ps, qq = rem - pp * ps;
        const float val = fminf(fmaxf(v[j], -1.0f), 1.0f);
        out[(c * H + hh * ps + pp) * W + ww * ps + qq] = val;
      }
      break;
    }
    case OASIS_EPI_GELU_TANH_FRAG: {
#pragma unroll
      for (int j = 0; j < 8; ++j) v[j] = gelu_tanh(v[j]);
      store8_bf16(e.out_bf16 + frag_index(m, n0, e.ld_out >> 5), v);
      break;
    }
    case OASIS_EPI_GELU_TANH_FP8: {
      // the 4 threads of one 32-column block are lanes 4i..4i+3 of the caller's loop
      float amax = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        v[j] = gelu_tanh(v[j]);
        amax = fmaxf(amax, fabsf(v[j]));
      }
      amax = quad_max(amax);
      const int sb = fp8_block_scale(amax);
      const float inv = fp8_block_inv(sb);
      *reinterpret_cast<uint2*>(e.out_fp8 + m * e.ld_out + n0) =
          make_uint2(pack4_fp8(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv),
                     pack4_fp8(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv));
      if ((n0 & 31) == 0) e.out_scale[m * e.ld_scale + (n0 >> 5)] = (uint8_t)sb;
      break;
    }
    default:
      break;
  }
}

// Rows of the QKV rotation tables a large-token workgroup copies to LDS for its epilogue (the
// cos rows, then the sin rows, each row ROPE_TP floats apart): the positions of a frame for the
// spatial tables, the frames of a stream for the temporal ones. 0 when the tables do not fit
// in tab_bytes (the epilogue then reads them from global memory). The 4-float pad puts the same
// dimension of consecutive positions 4 banks apart: a pass of the epilogue reads ~11 rows' tables
// at the same few dimensions, which a 64-float pitch sends to the same banks.
__device__ __forceinline__ int rope_lds_rows(const Epi& e, int M, int tab_bytes) {
  if (e.kind != OASIS_EPI_QKV_ROPE) return 0;
  // only positions some row m < M reaches: m % rows_per_frame, or its frame's index in the stream
  const int64_t frames = (M + e.rows_per_frame - 1) / e.rows_per_frame;
  const int64_t rows = e.rope_by_frame ? min(e.frames_per_stream, frames) : min(e.rows_per_frame, (int64_t)M);
  return rows * 2 * ROPE_TP * 4 <= tab_bytes ? (int)rows : 0;
}
// Workgroup-wide copy of those rows into tab (all threads of the workgroup call it).
__device__ __forceinline__ void rope_to_lds(const Epi& e, float* tab, int rows, int tid, int nthreads) {
  const int chunks = rows * 16;  // 16-byte chunks per table
  for (int i = tid; i < 2 * chunks; i += nthreads) {
    const int sel = i >= chunks, j = i - sel * chunks;
    const float* src = (sel ? e.rope_sinp : e.rope_cos) + j * 4;
    *reinterpret_cast<f32x4*>(tab + (sel * rows + (j >> 4)) * ROPE_TP + (j & 15) * 4) =
        *reinterpret_cast<const f32x4*>(src);
  }
}

Epi to_epi(const oasis_epilogue_t& x) {
  Epi e;
  e.kind = x.kind;
  e.n_heads = x.n_heads;
  e.bias = x.bias;
  e.out_f32 = x.out_f32;
  e.out_bf16 = static_cast<bf16*>(x.out_bf16);
  e.ld_out = x.ld_out;
  e.gate = x.gate;
  e.gate_fstride = x.gate_fstride;
  e.rows_per_frame = x.rows_per_frame > 0 ? x.rows_per_frame : 1;
  e.frames_per_stream = x.frames_per_stream > 0 ? x.frames_per_stream : 1;
  const DivMagic dr = div_magic((uint64_t)e.rows_per_frame), df = div_magic((uint64_t)e.frames_per_stream);
  e.rpf_magic = dr.magic;
  e.rpf_shift = dr.shift;
  e.fps_magic = df.magic;
  e.fps_shift = df.shift;
  e.q = static_cast<bf16*>(x.q);
  e.k = static_cast<bf16*>(x.k);
  e.v = static_cast<bf16*>(x.v);
  e.rope_cos = x.rope_cos;
  e.rope_sinp = x.rope_sinp;
  e.rope_by_frame = x.rope_by_frame;
  e.unpatch_grid_w = x.unpatch_grid_w;
  e.s_b = x.s_b;
  e.s_t = x.s_t;
  e.s_p = x.s_p;
  e.s_h = x.s_h;
  e.unpatch_patch = x.unpatch_patch;
  e.unpatch_channels = x.unpatch_channels;
  e.split_stride = x.split_stride;
  e.out_fp8 = static_cast<uint8_t*>(x.out_fp8);
  e.out_scale = static_cast<uint8_t*>(x.out_scale);
  e.ld_scale = x.ld_scale;
  e.mod_scale = x.mod_scale;
  e.mod_shift = x.mod_shift;
  e.ln_center = x.ln_center;
  e.ln_stats = x.ln_stats;
  e.ln_mod = static_cast<bf16*>(x.ln_mod);
  e.ln_eps = x.ln_eps;
  e.out_frag = x.out_frag;
  e.ln_group = 16;
  e.pf = oasis::prefetch_or_none(nullptr);
  return e;
}

// Checks the epilogue against the GEMM shape; returns OASIS_OK or an error code (message set).
inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check_epilogue(const Epi& e, int64_t M, int64_t N, int splits) {
  OASIS_REQUIRE(splits == 1 || e.kind == OASIS_EPI_PARTIAL_F32, OASIS_ERR_ARG,
                "gemm: split-K needs the PARTIAL_F32 epilogue");
  // the epilogue moves 16-byte vectors (8-byte e4m3 groups): every base pointer it touches must
  // be 16-byte aligned
  OASIS_REQUIRE(aligned16(e.bias) && aligned16(e.out_f32) && aligned16(e.out_bf16) && aligned16(e.gate) &&
                    aligned16(e.q) && aligned16(e.k) && aligned16(e.v) && aligned16(e.rope_cos) &&
                    aligned16(e.rope_sinp) && aligned16(e.out_fp8),
                OASIS_ERR_ARG, "gemm: epilogue pointers must be 16-byte aligned");
  switch (e.kind) {
    case OASIS_EPI_STORE_F32:
    case OASIS_EPI_GATED_RES:
    case OASIS_EPI_RESIDUAL:
    case OASIS_EPI_PARTIAL_F32:
      OASIS_REQUIRE(e.kind != OASIS_EPI_GATED_RES || e.rows_per_frame < (1ll << 31), OASIS_ERR_SHAPE,
                    "gemm: rows_per_frame too large");
      OASIS_REQUIRE(e.out_f32 && e.ld_out >= N && e.ld_out % 4 == 0, OASIS_ERR_ARG,
                    "gemm: fp32 epilogue needs out_f32 and ld_out >= N (multiple of 4)");
      OASIS_REQUIRE(e.kind != OASIS_EPI_GATED_RES || e.gate, OASIS_ERR_NULL, "gemm: gate is NULL");
      OASIS_REQUIRE(e.kind != OASIS_EPI_PARTIAL_F32 || splits == 1 || e.split_stride >= M * e.ld_out,
                    OASIS_ERR_ARG, "gemm: split_stride must be >= M * ld_out");
      break;
    case OASIS_EPI_STORE_BF16:
    case OASIS_EPI_GELU_TANH:
    case OASIS_EPI_GELU_ERF:
      OASIS_REQUIRE(e.out_bf16 && e.ld_out >= N && e.ld_out % 8 == 0, OASIS_ERR_ARG,
                    "gemm: bf16 epilogue needs out_bf16 and ld_out >= N (multiple of 8)");
      break;
    case OASIS_EPI_GELU_TANH_FRAG:
      OASIS_REQUIRE(e.out_bf16 && e.ld_out >= N && e.ld_out % 32 == 0 && M % 16 == 0, OASIS_ERR_ARG,
                    "gemm: GELU_TANH_FRAG needs out_bf16, ld_out >= N (multiple of 32) and M %% 16 == 0");
      break;
    case OASIS_EPI_GATED_RES_LN:
      OASIS_REQUIRE(e.rows_per_frame < (1ll << 31), OASIS_ERR_SHAPE, "gemm: rows_per_frame too large");
      OASIS_REQUIRE(e.out_f32 && e.out_bf16 && e.gate && e.mod_scale && e.mod_shift && e.ln_center && e.ln_stats &&
                        e.ln_mod,
                    OASIS_ERR_NULL, "gemm: GATED_RES_LN needs out_f32, out_bf16, gate, mod_scale, mod_shift, "
                                    "ln_center, ln_stats and ln_mod");
      OASIS_REQUIRE(aligned16(e.mod_scale) && aligned16(e.mod_shift) && aligned16(e.ln_mod) &&
                        ((uintptr_t)e.ln_stats & 7) == 0,
                    OASIS_ERR_ARG, "gemm: mod_scale, mod_shift and ln_mod must be 16-byte and ln_stats 8-byte aligned");
      OASIS_REQUIRE(e.ld_out == N && N % 32 == 0 && M % 16 == 0 && e.gate_fstride % 4 == 0, OASIS_ERR_ARG,
                    "gemm: GATED_RES_LN needs ld_out == N (a multiple of 32), M %% 16 == 0 and gate_fstride %% 4 == 0");
      OASIS_REQUIRE((M + e.rows_per_frame - 1) / e.rows_per_frame <= 8, OASIS_ERR_SHAPE,
                    "gemm: GATED_RES_LN covers at most 8 frames");
      break;
    case OASIS_EPI_GELU_TANH_LN:
      OASIS_REQUIRE(e.rows_per_frame < (1ll << 31), OASIS_ERR_SHAPE, "gemm: rows_per_frame too large");
      OASIS_REQUIRE(e.out_bf16 && e.ln_stats && e.ln_mod, OASIS_ERR_NULL,
                    "gemm: GELU_TANH_LN needs out_bf16, ln_stats and ln_mod");
      OASIS_REQUIRE(aligned16(e.ln_stats) && aligned16(e.ln_mod), OASIS_ERR_ARG,
                    "gemm: ln_stats and ln_mod must be 16-byte aligned");
      OASIS_REQUIRE(e.ld_out >= N && e.ld_out % (e.out_frag ? 32 : 8) == 0 && M % 16 == 0 && e.ln_eps >= 0.f,
                    OASIS_ERR_ARG, "gemm: GELU_TANH_LN needs ld_out >= N (a multiple of 32 in fragment order, "
                                   "else 8), M %% 16 == 0 and ln_eps >= 0");
      OASIS_REQUIRE((M + e.rows_per_frame - 1) / e.rows_per_frame <= 8, OASIS_ERR_SHAPE,
                    "gemm: GELU_TANH_LN covers at most 8 frames");
      break;
    case OASIS_EPI_GELU_TANH_FP8:
      OASIS_REQUIRE(e.out_fp8 && e.out_scale && N % 32 == 0 && e.ld_out >= N && e.ld_out % 8 == 0 &&
                        e.ld_scale >= N / 32,
                    OASIS_ERR_ARG, "gemm: GELU_TANH_FP8 needs out_fp8/out_scale, N %% 32 == 0, ld_out >= N "
                                   "(multiple of 8), ld_scale >= N/32");
      break;
    case OASIS_EPI_QKV_ROPE:
      OASIS_REQUIRE(e.rows_per_frame < (1ll << 31) && e.frames_per_stream < (1ll << 31), OASIS_ERR_SHAPE,
                    "gemm: rows_per_frame / frames_per_stream too large");
      OASIS_REQUIRE(e.q && e.k && e.v && e.rope_cos && e.rope_sinp, OASIS_ERR_NULL,
                    "gemm: QKV_ROPE needs q/k/v and rope tables");
      OASIS_REQUIRE(e.n_heads > 0 && N == 3LL * e.n_heads * 64, OASIS_ERR_SHAPE,
                    "gemm: QKV_ROPE needs N == 3*n_heads*64");
      {
        // the kernels address q, k and v with 32-bit element offsets
        const int64_t fr = (M + e.rows_per_frame - 1) / e.rows_per_frame;
        const int64_t streams = (fr + e.frames_per_stream - 1) / e.frames_per_stream;
        const int64_t last = (streams - 1) * e.s_b + (min(fr, e.frames_per_stream) - 1) * e.s_t +
                             (min(M, e.rows_per_frame) - 1) * e.s_p + (e.n_heads - 1) * e.s_h + 64;
        OASIS_REQUIRE(e.s_b >= 0 && e.s_t >= 0 && e.s_p >= 0 && e.s_h >= 0 && last < (1ll << 31), OASIS_ERR_SHAPE,
                      "gemm: QKV_ROPE offsets must be below 2^31 elements");
      }
      break;
    case OASIS_EPI_UNPATCHIFY:
      OASIS_REQUIRE(e.out_f32 && e.unpatch_patch > 0 && e.unpatch_grid_w > 0, OASIS_ERR_ARG,
                    "gemm: UNPATCHIFY needs out_f32, patch and grid_w");
      OASIS_REQUIRE(N == 3LL * e.unpatch_patch * e.unpatch_patch && e.rows_per_frame > 0 &&
                        M % e.rows_per_frame == 0 && e.rows_per_frame % e.unpatch_grid_w == 0,
                    OASIS_ERR_SHAPE, "gemm: UNPATCHIFY shape mismatch");
      break;
    default:
      OASIS_REQUIRE(false, OASIS_ERR_ARG, "gemm: unknown epilogue kind %d", e.kind);
  }
  return OASIS_OK;
}

}  // namespace
