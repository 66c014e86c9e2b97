// kv_rotate.h -- element codecs and the re-rotation kernels (contiguous,
// row-aligned, pair-task, element-wise LDS and grouped).
// Part of libdaser_kv: included by kv_move.hip, one translation unit.

#pragma once

#include "kv_page_kernels.h"

namespace {

// ---------------------------------------------------------------------------
// Element codecs for the rotation. Each 16-byte vector holds VE elements.

__device__ __forceinline__ float bf16_to_f32(uint32_t h) {
  return __uint_as_float(h << 16);
}
// Round-to-nearest-even fp32 -> bf16; NaN -> 0x7FC0 with its sign dropped.
__device__ __forceinline__ uint32_t f32_to_bf16(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}

__device__ __forceinline__ float fp16_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
// fp32 -> fp16 by the hardware conversion (round-to-nearest-even);
// NaN -> 0x7E00.
__device__ __forceinline__ uint32_t f32_to_fp16(float f) {
  if (__builtin_isnan(f)) return 0x7e00u;
  return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
}

// OCP e4m3fn (bias 7, no infinities, S.1111.111 = NaN) through the gfx950
// conversion instructions, which use the OCP formats: v_cvt_pk_f32_fp8
// decodes two codes, v_cvt_pk_fp8_f32 encodes two floats with
// round-to-nearest-even (both checked exhaustively against the bit-level
// definition on MI355X: all 256 codes, 200k values incl. every midpoint).
// Encoding saturates by clamping to +-448 first (compare-select keeps NaN);
// the instruction turns NaN into 0xFF, which the clamp range never produces,
// so 0xFF bytes are rewritten to the canonical 0x7F.
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float clamp448(float f) {
  f = f > 448.0f ? 448.0f : f;
  return f < -448.0f ? -448.0f : f;
}
// 0x80 in every byte of w that equals 0xFF.
__device__ __forceinline__ uint32_t ff_bytes(uint32_t w) {
  const uint32_t t = ~w;
  return ~(((t & 0x7f7f7f7fu) + 0x7f7f7f7fu) | t) & 0x80808080u;
}
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float* x) {
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)w, true);
  x[0] = lo.x;
  x[1] = lo.y;
  x[2] = hi.x;
  x[3] = hi.y;
}
__device__ __forceinline__ uint32_t f32x4_to_e4m3(const float* y) {
  int e = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(y[0]), clamp448(y[1]), 0, false);
  e = __builtin_amdgcn_cvt_pk_fp8_f32(clamp448(y[2]), clamp448(y[3]), e, true);
  const uint32_t w = (uint32_t)e;
  return w ^ ff_bytes(w);
}

// OCP e5m2 (bias 15, infinities, S.11111.{01,10,11} = NaN) through the
// gfx950 bf8 conversions (v_cvt_pk_f32_bf8 / v_cvt_pk_bf8_f32, round to
// nearest even). Encoding saturates as for e4m3: finite values and
// infinities clamp to +-57344 (compare-select keeps NaN), so an encoded byte
// with an all-ones exponent is NaN, rewritten to torch's canonical 0x7F.
__device__ __forceinline__ float clamp57344(float f) {
  f = f > 57344.0f ? 57344.0f : f;
  return f < -57344.0f ? -57344.0f : f;
}
__device__ __forceinline__ void e5m2x4_to_f32(uint32_t w, float* x) {
  const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, false);
  const f32x2 hi = __builtin_amdgcn_cvt_pk_f32_bf8((int)w, true);
  x[0] = lo.x;
  x[1] = lo.y;
  x[2] = hi.x;
  x[3] = hi.y;
}
__device__ __forceinline__ uint32_t f32x4_to_e5m2(const float* y) {
  int e = __builtin_amdgcn_cvt_pk_bf8_f32(clamp57344(y[0]), clamp57344(y[1]), 0, false);
  e = __builtin_amdgcn_cvt_pk_bf8_f32(clamp57344(y[2]), clamp57344(y[3]), e, true);
  const uint32_t w = (uint32_t)e;
  // bytes whose exponent bits (0x7C) are all set: 0x80 in each such byte
  const uint32_t x = (w & 0x7c7c7c7cu) ^ 0x7c7c7c7cu;  // zero byte <=> exponent all ones
  const uint32_t nan = ~(((x & 0x7f7f7f7fu) + 0x7f7f7f7fu) | x | 0x7f7f7f7fu);
  const uint32_t bytes = (nan >> 7) * 0xffu;
  return (w & ~bytes) | (0x7f7f7f7fu & bytes);
}

// The 8-bit formats: one byte per element, K scaled by the layer's k_scale.
template <int DT>
constexpr bool is_fp8() {
  return DT == DSR_DTYPE_FP8_E4M3 || DT == DSR_DTYPE_FP8_E5M2;
}

template <int DT>
struct Codec;

template <>
struct Codec<DSR_DTYPE_BF16> {
  static constexpr int VE = 8;
  __device__ static void decode(u32x4 v, float* x) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = bf16_to_f32(v[k] & 0xffffu);
      x[2 * k + 1] = bf16_to_f32(v[k] >> 16);
    }
  }
  __device__ static u32x4 encode(const float* y) {
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      v[k] = f32_to_bf16(y[2 * k]) | (f32_to_bf16(y[2 * k + 1]) << 16);
    return v;
  }
};

template <>
struct Codec<DSR_DTYPE_FP16> {
  static constexpr int VE = 8;
  __device__ static void decode(u32x4 v, float* x) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      x[2 * k] = fp16_to_f32(v[k] & 0xffffu);
      x[2 * k + 1] = fp16_to_f32(v[k] >> 16);
    }
  }
  __device__ static u32x4 encode(const float* y) {
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k)
      v[k] = f32_to_fp16(y[2 * k]) | (f32_to_fp16(y[2 * k + 1]) << 16);
    return v;
  }
};

template <>
struct Codec<DSR_DTYPE_FP8_E4M3> {
  static constexpr int VE = 16;
  __device__ static void decode(u32x4 v, float* x) {
#pragma unroll
    for (int k = 0; k < 4; ++k) e4m3x4_to_f32(v[k], x + 4 * k);
  }
  __device__ static u32x4 encode(const float* y) {
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = f32x4_to_e4m3(y + 4 * k);
    return v;
  }
};

template <>
struct Codec<DSR_DTYPE_FP8_E5M2> {
  static constexpr int VE = 16;
  __device__ static void decode(u32x4 v, float* x) {
#pragma unroll
    for (int k = 0; k < 4; ++k) e5m2x4_to_f32(v[k], x + 4 * k);
  }
  __device__ static u32x4 encode(const float* y) {
    u32x4 v;
#pragma unroll
    for (int k = 0; k < 4; ++k) v[k] = f32x4_to_e5m2(y + 4 * k);
    return v;
  }
};

struct RotArgs {
  UnitArgs u;
  const float2* cos_sin;
  const int32_t* rope_idx;
  int32_t n_tables;
  const int32_t* layer_group;  // per record layer: table block, -1 = no RoPE (null: all 0)
  int32_t n_groups;
  int32_t row_vecs;    // 16-byte vectors per K row (head_dim * e / 16)
  int32_t rot_half;    // rot_dim / 2 (pairs per row)
  int32_t task_vecs;   // rotation tasks per row
  int32_t tail_vec0;   // first un-rotated vector of a row
  int32_t tasks_per_row;
  int32_t rot_vecs;   // 16-byte vectors of a row inside the rotated region
  int32_t half_vecs;  // neox: vectors from a first-half vector to its partner
  const float* k_scale;
  // Pair-task kernel only: task columns per table column. 1 for token-major
  // K rows; block_size for the split-x K layout, where a row is one head's
  // [head_dim / X][block_size][X] block and vector c holds dims
  // (c / block_size) * X ... + X - 1 of token c % block_size.
  int32_t col_div = 1;
  // Contig and grouped kernels on split-x K pages (KX = true): head blocks
  // of 2^kx_row_shift vectors, block_size 2^kx_bs_shift, neox partners
  // kx_dist vectors apart (0 for gptj).
  int32_t kx_row_shift = 0;
  int32_t kx_bs_shift = 0;
  int32_t kx_dist = 0;
  // Grouped kernel: walk its groups in hardware dispatch order (consecutive
  // workgroups take consecutive groups) instead of XCD-contiguous eighths.
  int32_t hw_order = 0;
};

// Split-x K: the lane-consecutive vector index i of a page -> the vector it
// moves. Inside a head block the rotated region is walked in 64-vector runs
// whose lanes 0-31 take 32 consecutive first-half vectors and lanes 32-63
// their partners kx_dist vectors on, so a neox partner is always lane ^ 32
// and each half-wave still reads 512 contiguous bytes. Tail vectors (and all
// of gptj) keep their index. Needs kx_dist % 32 == 0 and 64 | block vectors.
__device__ __forceinline__ int kx_phys(const RotArgs& ra, int i) {
  const int q = i & ((1 << ra.kx_row_shift) - 1);
  if (q >= 2 * ra.kx_dist) return i;
  const int w = q & 63;
  return i - q + ((q >> 6) << 5) + (w & 31) + (w >= 32 ? ra.kx_dist : 0);
}

// Table column (dims c * VE ...) of physical K vector p: token-major rows
// have row_vecs vectors of consecutive dims; split-x head blocks hold
// block_size vectors per column.
template <bool KX>
__device__ __forceinline__ int k_column(const RotArgs& ra, int p) {
  return KX ? (p & ((1 << ra.kx_row_shift) - 1)) >> ra.kx_bs_shift : p % ra.row_vecs;
}

// Table of unit (page p, layer l): page p's delta table inside layer l's
// group block (cos_sin holds n_groups blocks of n_tables tables), or -1 when
// the page keeps its position or the layer has no RoPE (K copied as is).
__device__ __forceinline__ int rope_table(const RotArgs& ra, int64_t p, int l) {
  const int ti = ra.rope_idx[p];
  if (ti < 0 || ti >= ra.n_tables) return -1;
  if (!ra.layer_group) return ti;
  const int g = ra.layer_group[ra.u.layer0 + l];
  return g < 0 || g >= ra.n_groups ? -1 : g * ra.n_tables + ti;
}

// K-page rotation in rounds of kRotUnroll tasks per lane. Task t covers row
// t / tasks_per_row, column c = t % tasks_per_row:
//   neox, c < task_vecs: vector c of the rotated first half and its partner
//                        at +rot_half elements;
//   gptj, c < task_vecs: vector c, whose VE/2 adjacent pairs rotate in place;
//   c >= task_vecs:      one un-rotated 16-byte tail vector, copied.
// The table column of task column c is c / col_div (split-x K: the rows,
// columns and half distance are all counted in vectors of the head block).
template <int DT, int STYLE>
struct KRound {
  static constexpr int VE = Codec<DT>::VE;
  u32x4 a[kRotUnroll], b[kRotUnroll];
  int off[kRotUnroll];
  int kind[kRotUnroll];  // 0 = rotate, 1 = copy, -1 = none
  int c_of[kRotUnroll];

  __device__ __forceinline__ void load(const RotArgs& ra, rsrc_t rs, int base, int ntask,
                                       int row_bytes, int half_off) {
#pragma unroll
    for (int k = 0; k < kRotUnroll; ++k) {
      const int t = base + k * kThreads;
      kind[k] = -1;
      off[k] = 0;
      c_of[k] = 0;
      a[k] = u32x4{0u, 0u, 0u, 0u};
      b[k] = a[k];
      if (t < ntask) {
        const int row = t / ra.tasks_per_row;
        const int c = t - row * ra.tasks_per_row;
        c_of[k] = ra.col_div == 1 ? c : c / ra.col_div;
        if (c < ra.task_vecs) {
          kind[k] = 0;
          off[k] = row * row_bytes + (c << 4);
          a[k] = bload(rs, off[k]);
          if (STYLE == DSR_ROPE_NEOX) b[k] = bload(rs, off[k] + half_off);
        } else {
          kind[k] = 1;
          off[k] = row * row_bytes + ((ra.tail_vec0 + c - ra.task_vecs) << 4);
          a[k] = bload(rs, off[k]);
        }
      }
    }
  }

  __device__ __forceinline__ void store(rsrc_t rd, const float2* tab, int half_off,
                                        float scale, float inv_scale) {
    using C = Codec<DT>;
    constexpr bool kScaled = is_fp8<DT>();
#pragma unroll
    for (int k = 0; k < kRotUnroll; ++k) {
      if (kind[k] == 1) {
        bstore(rd, off[k], a[k]);
      } else if (kind[k] == 0) {
        float x[VE];
        C::decode(a[k], x);
        if (STYLE == DSR_ROPE_NEOX) {
          float z[VE];
          C::decode(b[k], z);
          const int j0 = c_of[k] * VE;
#pragma unroll
          for (int e = 0; e < VE; ++e) {
            const float2 cs = tab[j0 + e];
            const float x1 = kScaled ? x[e] * scale : x[e];
            const float x2 = kScaled ? z[e] * scale : z[e];
            const float y1 = x1 * cs.x - x2 * cs.y;
            const float y2 = x2 * cs.x + x1 * cs.y;
            x[e] = kScaled ? y1 * inv_scale : y1;
            z[e] = kScaled ? y2 * inv_scale : y2;
          }
          bstore(rd, off[k], C::encode(x));
          bstore(rd, off[k] + half_off, C::encode(z));
        } else {
          const int j0 = c_of[k] * (VE / 2);
#pragma unroll
          for (int e = 0; e < VE / 2; ++e) {
            const float2 cs = tab[j0 + e];
            const float x1 = kScaled ? x[2 * e] * scale : x[2 * e];
            const float x2 = kScaled ? x[2 * e + 1] * scale : x[2 * e + 1];
            const float y1 = x1 * cs.x - x2 * cs.y;
            const float y2 = x2 * cs.x + x1 * cs.y;
            x[2 * e] = kScaled ? y1 * inv_scale : y1;
            x[2 * e + 1] = kScaled ? y2 * inv_scale : y2;
          }
          bstore(rd, off[k], C::encode(x));
        }
      }
    }
  }
};

// One page_bytes run copied in rounds of U vectors per lane.
template <int U>
struct VRound {
  u32x4 r[U];
  __device__ __forceinline__ void load(rsrc_t rs, int base, int nvec) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + k * kThreads;
      r[k] = i < nvec ? bload(rs, i << 4) : u32x4{0u, 0u, 0u, 0u};
    }
  }
  __device__ __forceinline__ void store(rsrc_t rd, int base, int nvec) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + k * kThreads;
      if (i < nvec) bstore(rd, i << 4, r[k]);
    }
  }
  // head-major cache page: vector i of the round goes to cache vector hnd_vec(i)
  __device__ __forceinline__ void store_hnd(const UnitArgs& a, rsrc_t rd, int base, int nvec) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + k * kThreads;
      if (i < nvec) bstore(rd, hnd_vec(a, i) << 4, r[k]);
    }
  }
  // K of a split-x page: vector i of the round is physical vector kx_phys(i)
  __device__ __forceinline__ void load_kx(const RotArgs& ra, rsrc_t rs, int base, int nvec) {
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + k * kThreads;
      r[k] = i < nvec ? bload(rs, kx_phys(ra, i) << 4) : u32x4{0u, 0u, 0u, 0u};
    }
  }
};

// One workgroup per (page, layer) unit in page-list order. V, and K of pages
// without a table (rope_idx < 0), are copied bit-exactly; K of the others is
// re-rotated row by row with the page's (cos, sin) table staged in LDS. The
// first round of V and K loads is issued before the table is fetched and the
// workgroup synchronises, so the table latency overlaps the page reads.
template <int DT, int STYLE>
__global__ __launch_bounds__(kThreads) void kv_scatter_rerotate_kernel(RotArgs ra) {
  __shared__ float2 tab[kMaxRotHalf];
  uint8_t *cache, *rec;
  int l;
  // ra.u.parts consecutive workgroups share a unit (large pages), each
  // moving a part of whole rows of both runs
  const int parts = ra.u.parts;
  const int64_t w = xcd_unit(ra.u.n_units * parts);
  if (w < 0) return;
  const int64_t vu = parts > 1 ? udiv32(w, parts) : w;
  const int64_t u = layer_major_of(vu, ra.u.n_units, ra.u.n_layers);
  if (!unit_addresses(ra.u, u, &cache, &rec, &l)) return;
  const int64_t p = udiv32(u, ra.u.n_layers);
  const int ti = rope_table(ra, p, l);
  const int64_t pb = ra.u.page_bytes / parts;
  const int64_t po = pb * (w - vu * parts);
  uint8_t* const vrec = rec + ra.u.page_bytes + po;
  uint8_t* const vcache = cache + ra.u.kv_stride + po;
  rec += po;
  cache += po;
  if (ti < 0) {
    copy_halves<kRotCopyUnroll>(rec, vrec, cache, vcache, pb);
    return;
  }
  const rsrc_t ks = make_rsrc(rec, pb), kd = make_rsrc(cache, pb);
  const rsrc_t vs = make_rsrc(vrec, pb), vd = make_rsrc(vcache, pb);
  const int nvec = (int)(pb >> 4);
  const int row_bytes = ra.row_vecs << 4;
  const int ntask = (int)(pb / row_bytes) * ra.tasks_per_row;
  const int half_off = ra.rot_half * 16 / Codec<DT>::VE * ra.col_div;

  VRound<kScatterUnroll> v;
  KRound<DT, STYLE> k;
  v.load(vs, threadIdx.x, nvec);
  k.load(ra, ks, threadIdx.x, ntask, row_bytes, half_off);

  const float2* src_tab = ra.cos_sin + (int64_t)ti * ra.rot_half;
  for (int j = threadIdx.x; j < ra.rot_half; j += kThreads) tab[j] = src_tab[j];
  float scale = 1.0f, inv_scale = 1.0f;
  if (is_fp8<DT>()) {
    scale = ra.k_scale[ra.u.layer0 + l];
    inv_scale = 1.0f / scale;
  }
  __syncthreads();

  v.store(vd, threadIdx.x, nvec);
  k.store(kd, tab, half_off, scale, inv_scale);
  for (int base = threadIdx.x + kThreads * kScatterUnroll; base < nvec;
       base += kThreads * kScatterUnroll) {
    v.load(vs, base, nvec);
    v.store(vd, base, nvec);
  }
  for (int base = threadIdx.x + kThreads * kRotUnroll; base < ntask;
       base += kThreads * kRotUnroll) {
    k.load(ra, ks, base, ntask, row_bytes, half_off);
    k.store(kd, tab, half_off, scale, inv_scale);
  }
}

// One K vector after rotation: c is its vector column in the row, own its
// bytes, partner (neox) the bytes of the vector half a rotation away.
// Vectors past the rotated region are returned unchanged.
template <int DT, int STYLE>
__device__ __forceinline__ u32x4 rotate_vec(const RotArgs& ra, u32x4 own, u32x4 partner, int c,
                                            const float2* tab, float scale, float inv_scale) {
  using C = Codec<DT>;
  constexpr int VE = C::VE;
  constexpr bool kScaled = is_fp8<DT>();
  if (c >= ra.rot_vecs) return own;
  float x[VE];
  C::decode(own, x);
  if (STYLE == DSR_ROPE_NEOX) {
    float z[VE];
    C::decode(partner, z);
    const bool first = c < ra.half_vecs;
    const int j0 = (first ? c : c - ra.half_vecs) * VE;
    const float sg = first ? -1.0f : 1.0f;
#pragma unroll
    for (int e = 0; e < VE; ++e) {
      const float2 cs = tab[j0 + e];
      const float xo = kScaled ? x[e] * scale : x[e];
      const float xp = kScaled ? z[e] * scale : z[e];
      // first half: x c - p s; second half: x c + p s
      const float y = xo * cs.x + sg * (xp * cs.y);
      x[e] = kScaled ? y * inv_scale : y;
    }
  } else {
    const int j0 = c * (VE / 2);
#pragma unroll
    for (int e = 0; e < VE / 2; ++e) {
      const float2 cs = tab[j0 + e];
      const float x1 = kScaled ? x[2 * e] * scale : x[2 * e];
      const float x2 = kScaled ? x[2 * e + 1] * scale : x[2 * e + 1];
      const float y1 = x1 * cs.x - x2 * cs.y;
      const float y2 = x2 * cs.x + x1 * cs.y;
      x[2 * e] = kScaled ? y1 * inv_scale : y1;
      x[2 * e + 1] = kScaled ? y2 * inv_scale : y2;
    }
  }
  return C::encode(x);
}

// Contiguous variant: lane-consecutive 16-byte vectors over the whole K page
// (every load instruction of a wave covers 1 KiB of contiguous page), with
// the neox partner vector fetched from lane ^ half_vecs by a cross-lane
// shuffle. Valid when half_vecs is a power of two <= 32 dividing the row
// evenly (rows then start on 2*half_vecs lane boundaries), and always for
// gptj, whose pairs sit inside one vector.
template <int DT, int STYLE, int U, bool KX, bool HND = false>
__device__ __forceinline__ void rotate_contig_round(const RotArgs& ra, VRound<U>& kk,
                                                    int base, int nvec, rsrc_t kd,
                                                    const float2* tab, float scale,
                                                    float inv_scale) {
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int i = base + k * kThreads;
    u32x4 q = kk.r[k];
    if (STYLE == DSR_ROPE_NEOX) {  // whole wave takes part in the shuffle
      const int dist = KX ? 32 : ra.half_vecs;
#pragma unroll
      for (int w = 0; w < 4; ++w) q[w] = (unsigned)__shfl_xor((int)kk.r[k][w], dist);
    }
    if (i >= nvec) continue;
    // split-x: both sides move vector kx_phys(i); head-major: the record
    // row order is token-major (the table column follows i), the cache's not
    const int p = KX ? kx_phys(ra, i) : i;
    bstore(kd, (HND ? hnd_vec(ra.u, i) : p) << 4,
           rotate_vec<DT, STYLE>(ra, kk.r[k], q, k_column<KX>(ra, p), tab, scale, inv_scale));
  }
}

// K and V vectors per lane per round: one round covers a 32 KiB bf16 or a
// 16 KiB e4m3 Llama page.
template <int DT>
constexpr int rot_contig_unroll() {
  return is_fp8<DT>() ? 4 : 8;
}

template <int DT, int STYLE, bool KX, bool HND = false>
__global__ __launch_bounds__(kThreads) void kv_scatter_rerotate_contig_kernel(RotArgs ra) {
  __shared__ float2 tab[kMaxRotHalf];
  uint8_t *cache, *rec;
  int l;
  const int64_t u = layer_major_unit(ra.u.n_units, ra.u.n_layers);
  if (u < 0 || !unit_addresses(ra.u, u, &cache, &rec, &l)) return;
  const int64_t p = udiv32(u, ra.u.n_layers);
  const int ti = rope_table(ra, p, l);
  const int64_t pb = ra.u.page_bytes;
  if (ti < 0) {
    if (HND)
      copy_halves_hnd<kRotCopyUnroll, false>(ra.u, cache, rec);
    else
      copy_halves<kRotCopyUnroll>(rec, rec + pb, cache, cache + ra.u.kv_stride, pb);
    return;
  }
  constexpr int U = rot_contig_unroll<DT>();
  const rsrc_t ks = make_rsrc(rec, pb), kd = make_rsrc(cache, pb);
  const rsrc_t vs = make_rsrc(rec + pb, pb), vd = make_rsrc(cache + ra.u.kv_stride, pb);
  const int nvec = (int)(pb >> 4);
  VRound<U> v, kk;
  v.load(vs, threadIdx.x, nvec);
  if (KX)
    kk.load_kx(ra, ks, threadIdx.x, nvec);
  else
    kk.load(ks, threadIdx.x, nvec);
  const float2* src_tab = ra.cos_sin + (int64_t)ti * ra.rot_half;
  for (int j = threadIdx.x; j < ra.rot_half; j += kThreads) tab[j] = src_tab[j];
  float scale = 1.0f, inv_scale = 1.0f;
  if (is_fp8<DT>()) {
    scale = ra.k_scale[ra.u.layer0 + l];
    inv_scale = 1.0f / scale;
  }
  __syncthreads();
  const int rounds = (nvec + kThreads * U - 1) / (kThreads * U);
  for (int r = 0; r < rounds; ++r) {  // uniform trip count: shuffles stay converged
    const int base = r * kThreads * U + threadIdx.x;
    if (r > 0) {
      v.load(vs, base, nvec);
      if (KX)
        kk.load_kx(ra, ks, base, nvec);
      else
        kk.load(ks, base, nvec);
    }
    if (HND)
      v.store_hnd(ra.u, vd, base, nvec);
    else
      v.store(vd, base, nvec);
    rotate_contig_round<DT, STYLE, U, KX, HND>(ra, kk, base, nvec, kd, tab, scale, inv_scale);
  }
}

// neox rows whose partner distance is not a power of two (head_dim 80, 96,
// 192, ...): each wave takes rpw = 64 / row_vecs whole rows (lanes past
// rpw * row_vecs idle), so a vector's partner half a rotation away lies in
// the same wave and comes from lane +- half_vecs by an arbitrary-lane
// shuffle. Idle lanes and rows past the page get an offset beyond the
// descriptor: their loads read 0 and their stores are dropped. One unit per
// workgroup, layer-major; V is copied in flat rounds alongside. Replaced the
// pair-task kernel for these shapes (3.5-4.2 TB/s, 35-45% behind a plain
// scatter of the same pages).
template <int DT>
__global__ __launch_bounds__(kThreads) void kv_scatter_rerotate_rows_kernel(RotArgs ra) {
  constexpr int U = rot_contig_unroll<DT>();
  __shared__ float2 tab[kMaxRotHalf];
  uint8_t *cache, *rec;
  int l;
  // ra.u.parts consecutive workgroups share a unit (large pages), each
  // moving a part of whole rows of both runs
  const int parts = ra.u.parts;
  const int64_t w = xcd_unit(ra.u.n_units * parts);
  if (w < 0) return;
  const int64_t vu = parts > 1 ? udiv32(w, parts) : w;
  const int64_t u = layer_major_of(vu, ra.u.n_units, ra.u.n_layers);
  if (!unit_addresses(ra.u, u, &cache, &rec, &l)) return;
  const int64_t p = udiv32(u, ra.u.n_layers);
  const int ti = rope_table(ra, p, l);
  const int64_t pb = ra.u.page_bytes / parts;
  const int64_t po = pb * (w - vu * parts);
  uint8_t* const vrec = rec + ra.u.page_bytes + po;
  uint8_t* const vcache = cache + ra.u.kv_stride + po;
  rec += po;
  cache += po;
  if (ti < 0) {
    copy_halves<kRotCopyUnroll>(rec, vrec, cache, vcache, pb);
    return;
  }
  const rsrc_t ks = make_rsrc(rec, pb), kd = make_rsrc(cache, pb);
  const rsrc_t vs = make_rsrc(vrec, pb), vd = make_rsrc(vcache, pb);
  const int nvec = (int)(pb >> 4);
  const int rv = ra.row_vecs;
  const int rpw = kWave / rv;
  const int rows = nvec / rv;
  const int slots = (rows + rpw - 1) / rpw;  // wave-sized groups of rows
  const int lane = (int)threadIdx.x % kWave;
  const int wave = (int)threadIdx.x / kWave;
  const int r_in = lane / rv;
  const int c = lane - r_in * rv;
  const int h = ra.half_vecs;
  const int partner = c < h ? lane + h : c < 2 * h ? lane - h : lane;
  const int waves = kThreads / kWave;
  const int rounds_k = (slots + waves * U - 1) / (waves * U);
  const int rounds_v = (nvec + kThreads * U - 1) / (kThreads * U);
  const int rounds = rounds_k > rounds_v ? rounds_k : rounds_v;
  auto k_off = [&](int r, int k) {
    const int row = ((r * U + k) * waves + wave) * rpw + r_in;
    return r_in < rpw && row < rows ? (row * rv + c) << 4 : (int)pb;
  };
  VRound<U> v;
  u32x4 x[U];
  v.load(vs, threadIdx.x, nvec);
#pragma unroll
  for (int k = 0; k < U; ++k) x[k] = bload(ks, k_off(0, k));
  const float2* src_tab = ra.cos_sin + (int64_t)ti * ra.rot_half;
  for (int j = threadIdx.x; j < ra.rot_half; j += kThreads) tab[j] = src_tab[j];
  float scale = 1.0f, inv_scale = 1.0f;
  if (is_fp8<DT>()) {
    scale = ra.k_scale[ra.u.layer0 + l];
    inv_scale = 1.0f / scale;
  }
  __syncthreads();
  for (int r = 0; r < rounds; ++r) {  // uniform trip count: shuffles stay converged
    const int base = r * kThreads * U + threadIdx.x;
    if (r > 0) {
      v.load(vs, base, nvec);
#pragma unroll
      for (int k = 0; k < U; ++k) x[k] = bload(ks, k_off(r, k));
    }
    v.store(vd, base, nvec);
#pragma unroll
    for (int k = 0; k < U; ++k) {
      u32x4 q;
#pragma unroll
      for (int w = 0; w < 4; ++w) q[w] = (unsigned)__shfl((int)x[k][w], partner);
      bstore(kd, k_off(r, k),
             rotate_vec<DT, DSR_ROPE_NEOX>(ra, x[k], q, c, tab, scale, inv_scale));
    }
  }
}

// Any even rot_dim and either style, for rotary widths that do not fill
// whole 16-byte vectors (partial rotary of 24 or 20 dims, ...). A chunk of
// the page's K rows is staged in LDS; each lane decodes one output vector,
// rotates its elements below rot_dim with partners read element by element
// from LDS (a neox partner may straddle vectors), re-encodes, and keeps the
// raw bits of the elements at or past rot_dim through a bit mask. One unit
// per workgroup, layer-major; V is copied alongside.
template <int DT>
__device__ __forceinline__ float elem_decode(uint32_t bits) {
  if (DT == DSR_DTYPE_BF16) return bf16_to_f32(bits);
  if (DT == DSR_DTYPE_FP16) return fp16_to_f32(bits);
  if (DT == DSR_DTYPE_FP8_E5M2) return __builtin_amdgcn_cvt_pk_f32_bf8((int)bits, false)[0];
  return __builtin_amdgcn_cvt_pk_f32_fp8((int)bits, false)[0];
}

template <int DT, int STYLE>
__global__ __launch_bounds__(kThreads) void kv_scatter_rerotate_lds_kernel(RotArgs ra) {
  using C = Codec<DT>;
  constexpr int VE = C::VE;
  constexpr int EB = is_fp8<DT>() ? 8 : 16;  // bits per element
  constexpr int PER = 32 / EB;                           // elements per dword
  constexpr bool kScaled = is_fp8<DT>();
  constexpr int kChunkVecs = 2048;  // 32 KiB of K rows per pass
  __shared__ u32x4 buf[kChunkVecs];
  __shared__ float2 tab[kMaxRotHalf];
  uint8_t *cache, *rec;
  int l;
  // ra.u.parts consecutive workgroups share a unit (large pages), each
  // moving a part of whole rows of both runs
  const int parts = ra.u.parts;
  const int64_t w = xcd_unit(ra.u.n_units * parts);
  if (w < 0) return;
  const int64_t vu = parts > 1 ? udiv32(w, parts) : w;
  const int64_t u = layer_major_of(vu, ra.u.n_units, ra.u.n_layers);
  if (!unit_addresses(ra.u, u, &cache, &rec, &l)) return;
  const int64_t p = udiv32(u, ra.u.n_layers);
  const int ti = rope_table(ra, p, l);
  const int64_t pb = ra.u.page_bytes / parts;
  const int64_t po = pb * (w - vu * parts);
  uint8_t* const vrec = rec + ra.u.page_bytes + po;
  uint8_t* const vcache = cache + ra.u.kv_stride + po;
  rec += po;
  cache += po;
  if (ti < 0) {
    copy_halves<kRotCopyUnroll>(rec, vrec, cache, vcache, pb);
    return;
  }
  const rsrc_t ks = make_rsrc(rec, pb), kd = make_rsrc(cache, pb);
  const rsrc_t vs = make_rsrc(vrec, pb), vd = make_rsrc(vcache, pb);
  const int nvec = (int)(pb >> 4);
  {
    VRound<kRotCopyUnroll> v;  // V: a plain copy
    for (int base = threadIdx.x; base < nvec; base += kThreads * kRotCopyUnroll) {
      v.load(vs, base, nvec);
      v.store(vd, base, nvec);
    }
  }
  const float2* src_tab = ra.cos_sin + (int64_t)ti * ra.rot_half;
  for (int j = threadIdx.x; j < ra.rot_half; j += kThreads) tab[j] = src_tab[j];
  float scale = 1.0f, inv_scale = 1.0f;
  if (kScaled) {
    scale = ra.k_scale[ra.u.layer0 + l];
    inv_scale = 1.0f / scale;
  }
  const uint32_t* bw = reinterpret_cast<const uint32_t*>(buf);
  const int rv = ra.row_vecs, half = ra.rot_half, rot = 2 * ra.rot_half;
  const int rows = nvec / rv, rpc = kChunkVecs / rv;
  for (int r0 = 0; r0 < rows; r0 += rpc) {
    const int nv = (rows - r0 < rpc ? rows - r0 : rpc) * rv;
    __syncthreads();  // the previous chunk's readers are done (and the table is in)
    for (int i = threadIdx.x; i < nv; i += kThreads) buf[i] = bload(ks, (r0 * rv + i) << 4);
    __syncthreads();
    for (int i = threadIdx.x; i < nv; i += kThreads) {
      const int row = i / rv, c = i - row * rv;
      const u32x4 own = buf[i];
      float x[VE];
      C::decode(own, x);
      u32x4 mask = u32x4{0u, 0u, 0u, 0u};
#pragma unroll
      for (int e = 0; e < VE; ++e) {
        const int j = c * VE + e;
        if (j >= rot) continue;
        int pj, jj;
        float sg;
        if (STYLE == DSR_ROPE_NEOX) {
          const bool first = j < half;
          pj = first ? j + half : j - half;
          jj = first ? j : j - half;
          sg = first ? -1.0f : 1.0f;
        } else {
          pj = j ^ 1;
          jj = j >> 1;
          sg = (j & 1) ? 1.0f : -1.0f;
        }
        const int pe = pj % VE;
        const uint32_t word = bw[(row * rv + pj / VE) * 4 + pe / PER];
        const float pv = elem_decode<DT>((word >> (EB * (pe % PER))) & ((1u << EB) - 1u));
        const float2 cs = tab[jj];
        const float xo = kScaled ? x[e] * scale : x[e];
        const float xp = kScaled ? pv * scale : pv;
        const float y = xo * cs.x + sg * (xp * cs.y);
        x[e] = kScaled ? y * inv_scale : y;
        mask[e / PER] |= ((1u << EB) - 1u) << (EB * (e % PER));
      }
      const u32x4 enc = C::encode(x);
      bstore(kd, (r0 * rv + i) << 4, (enc & mask) | (own & ~mask));
    }
  }
}

// Re-rotation over G units per workgroup (layer-major order, as the one-unit
// kernel). The group's (cos, sin) tables are staged in LDS, one rot_half
// stretch per unit; G * rot_half <= kMaxRotHalf. K of an un-rotated unit is
// stored as loaded.
template <int DT, int STYLE, bool KX, bool HND = false>
__global__ __launch_bounds__(kThreads) void kv_scatter_rerotate_grouped_kernel(RotArgs ra,
                                                                               int G) {
  constexpr int U = rot_contig_unroll<DT>();
  __shared__ float2 tab[kMaxRotHalf];
  const UnitArgs& a = ra.u;
  // a.parts > 1 (with G = 1, token-major pages): a.parts consecutive
  // workgroups share a unit, each moving one part of its K and V runs
  const int64_t ng = udiv32(a.n_units * a.parts + G - 1, G);
  const int64_t gw = ra.hw_order ? ((int64_t)blockIdx.x < ng ? (int64_t)blockIdx.x : -1)
                                 : xcd_unit(ng);
  if (gw < 0) return;
  const int64_t g = a.parts > 1 ? udiv32(gw, a.parts) : gw;
  const int64_t pbytes = a.parts > 1 ? a.page_bytes / a.parts : a.page_bytes;
  const int64_t pofs = a.parts > 1 ? pbytes * (gw - g * a.parts) : 0;
  const int64_t n_pages = udiv32(a.n_units, a.n_layers);
  const int nvec = (int)(pbytes >> 4);
  int64_t p0;
  int l0;
  const int64_t n_here = group_start<false>(a, g, G, n_pages, &p0, &l0);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int lane = (int)threadIdx.x % kWave;
  rsrc_t kd[U], vd[U];
  u32x4 rk[U], rv[U];
  int tj[U];    // LDS table slot of the vector's unit (-1: copy)
  float sc[U];  // its layer's K scale (e4m3)
  int off[U];
  int koff[U];  // K: split-x pages move vector kx_phys(i) in lane slot i
  int coff[U];  // cache-side offset of record vector i (head-major: hnd_vec)
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int fw = k * kThreads + wave * kWave;
    const int j = fw / nvec;
    off[k] = (fw - j * nvec + lane) << 4;
    koff[k] = KX ? kx_phys(ra, off[k] >> 4) << 4 : off[k];
    coff[k] = HND ? hnd_vec(a, off[k] >> 4) << 4 : koff[k];
    const UnitRsrc u = unit_rsrc<false>(a, n_pages, p0, l0, j, n_here);
    const int64_t un = u.n ? pbytes : 0;
    rk[k] = bload(make_rsrc(u.rec + pofs, un), koff[k]);
    rv[k] = bload(make_rsrc(u.rec + a.page_bytes + pofs, un), off[k]);
    kd[k] = make_rsrc(u.cache + pofs, un);
    vd[k] = make_rsrc(u.cache + a.kv_stride + pofs, un);
    tj[k] = u.n && rope_table(ra, u.p, u.l) >= 0 ? j : -1;
    sc[k] = is_fp8<DT>() && u.n ? ra.k_scale[a.layer0 + u.l] : 1.0f;
  }
  // tables of the group's units, fetched while the page loads are in flight
  for (int e = threadIdx.x; e < (int)n_here * ra.rot_half; e += kThreads) {
    const int jj = e / ra.rot_half;
    int64_t p;
    int l;
    unit_at<false>(a, n_pages, p0, l0, jj, &p, &l);
    const int ti = rope_table(ra, p, l);
    if (ti >= 0) tab[e] = ra.cos_sin[(int64_t)ti * ra.rot_half + (e - jj * ra.rot_half)];
  }
#pragma unroll
  for (int k = 0; k < U; ++k) bstore(vd[k], HND ? coff[k] : off[k], rv[k]);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < U; ++k) {
    u32x4 q = rk[k];
    if (STYLE == DSR_ROPE_NEOX) {
      const int dist = KX ? 32 : ra.half_vecs;
#pragma unroll
      for (int x = 0; x < 4; ++x) q[x] = (unsigned)__shfl_xor((int)rk[k][x], dist);
    }
    const int t = tj[k] < 0 ? 0 : tj[k];
    const u32x4 r = rotate_vec<DT, STYLE>(ra, rk[k], q, k_column<KX>(ra, koff[k] >> 4),
                                          tab + t * ra.rot_half, sc[k], 1.0f / sc[k]);
    bstore(kd[k], coff[k], tj[k] < 0 ? rk[k] : r);
  }
}

}  // namespace
