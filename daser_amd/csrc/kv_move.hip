// kv_move.hip -- gfx950 kernels and C ABI for DaseR's KV data-movement path.
//
// Three operations, all HBM-bandwidth bound (no contraction, no MFMA):
//   dsr_gather            paged block cache  -> contiguous slot records
//   dsr_scatter           slot records       -> paged block cache
//   dsr_scatter_rerotate  slot records       -> paged block cache, with the K
//                         half of selected pages rotated by a RoPE position
//                         delta in fp32 on the way through.
//
// Work decomposition. A vLLM page (block_size tokens x H heads x D dims) is
// contiguous inside each per-layer cache; only the block index is permuted.
// The unit of work is therefore one (page, layer): two contiguous runs of
// page_bytes (K and V) on each side. One 256-lane workgroup owns one unit and
// moves it with 16-byte lane vectors (buffer_load_dwordx4 /
// buffer_store_dwordx4 through a descriptor bounded to the run), issuing
// every load of a round before any store so each lane keeps up to 2*U
// 16-byte requests in flight. No LDS is needed for the copy: both sides are
// contiguous within a unit. The re-rotation kernels keep the unit's
// (cos, sin) table in LDS.
//
// Kernel choice, by page and row geometry (all inside the entry points):
//   gather / scatter: one unit per workgroup; pages of at most 4 KiB
//     (scatter) or under 4 KiB (gather) take several units per workgroup
//     (kv_copy_grouped_kernel).
//   re-rotation: kv_scatter_rerotate_grouped_kernel for pages below U * 4
//     KiB and 16-bit pages of exactly U * 4 KiB; kv_scatter_rerotate_contig_
//     kernel for larger pages with a power-of-two partner distance;
//     kv_scatter_rerotate_rows_kernel for other neox rows of <= 64 vectors;
//     the pair-task kv_scatter_rerotate_kernel otherwise.
//   token form (dsr_gather_slots / dsr_scatter_slots): kv_slots_small_kernel
//     for rows of <= 32 vectors, kv_slots_kernel above.
// Calls too large for one launch run as several over page (token) ranges.
//
// Reference being replaced: the Python per-(request, block, layer) torch
// copy_ loops of daser/connector/daser_connector.py:536-551 (load) and
// :610-632 (save).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "daser_kv.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;     // 4 wave64 per workgroup
constexpr int kWave = 64;
constexpr int kMaxGroup = 64;     // units per workgroup of the grouped copy kernels
constexpr int kGatherUnroll = 16;  // 16-byte vectors per lane per half per round
constexpr int kScatterUnroll = 16;
constexpr int kRotCopyUnroll = 8;  // copy of unrotated pages inside the re-rotation kernels
constexpr int kRotUnroll = 4;      // rotation tasks per lane per round (pair-task kernel)
// Workgroups per CU for the re-rotation kernel, applied with dynamic LDS
// sized from the CU's LDS capacity (env DSR_ROT_WG_PER_CU overrides, for
// tuning). Measured in-process at the Llama-3-8B shapes: 16-bit K (64 KiB
// per unit) runs best at 2-3 per CU (7.67 ms vs 7.87 ms at 4-8 and 11.0 ms
// at 1); e4m3 (32 KiB per unit) at 4 per CU (24.17 ms; 24.4-24.5 ms at 6-12,
// 30.1 ms at 2).
template <int DT>
constexpr int rot_wg_per_cu() {
  return DT == DSR_DTYPE_FP8_E4M3 ? 4 : 2;
}
// The same for the grouped re-rotation kernel (pages below U * 4 KiB; env
// DSR_ROT_GROUPED_WG_PER_CU overrides). Measured in-process at the
// Llama-3-70B TP8 share: 16-bit K 6.97 ms at 4 per CU (7.41 at 2, 7.07 at
// 8); e4m3 with 2 KiB pages 3.24 ms at 8 per CU (3.56 at 4), with 8 KiB
// pages 12.96 ms at 8 (13.72 at 4).
template <int DT>
constexpr int rot_grouped_wg_per_cu() {
  return DT == DSR_DTYPE_FP8_E4M3 ? 8 : 4;
}
// The grouped kernel with one unit per workgroup (16-bit pages of exactly
// U * 4 KiB, the Llama-3-8B/70B shapes): 3 per CU. Measured in-process:
// config 3 7.05 ms at 2-3 per CU, 7.36 at 4-5 (the contig kernel 7.68);
// config 5 55.1 ms at 2-3, 50.4 at 4-6 (contig 55.4), where the shared
// source chunks' reads hit the memory-side cache. 3 is taken for the
// HBM-bound case. e4m3 keeps the contig kernel (24.05 vs 24.22 ms at
// config 4).
constexpr int kRotSingleWgPerCu = 3;
constexpr int kMaxRotHalf = 512;   // LDS table capacity: rot_dim <= 1024
constexpr int kXcds = 8;           // MI355X: 8 XCDs, workgroups dealt round-robin

// Cache-policy bits of gfx950 buffer instructions (CPol: sc0 = 1, nt = 2,
// sc1 = 16). Loads stream through (nt); stores are written with sc0 sc1,
// which measured fastest for these write-once streams (6.0 vs 5.2 TB/s for
// default-policy stores at the Llama-3-8B shape).
constexpr int kLoadPolicy = 2;
constexpr int kStorePolicy = 17;
// Buffer descriptor word 3 for raw (untyped) dword access on CDNA3/4.
constexpr int kRsrcWord3 = 0x00020000;

struct UnitArgs {
  const uint64_t* layer_base;
  int64_t kv_stride;
  int64_t page_stride;
  int64_t page_bytes;
  int64_t num_blocks;
  const int32_t* page_ids;
  const int64_t* slot_offsets;
  uint8_t* staging;
  int64_t staging_bytes;
  int64_t layer_bytes;
  int64_t n_units;
  int32_t n_layers;
  int32_t layer0;
};

// Workgroup -> unit. Hardware deals consecutive workgroup ids round-robin
// over the 8 XCDs; remapping so that each XCD walks one contiguous eighth of
// the unit list keeps each XCD's stream of records contiguous (measured
// +2% over the identity mapping for the gather). Returns -1 past the end.
__device__ __forceinline__ int64_t xcd_unit(int64_t n_units) {
  const int64_t per = (n_units + kXcds - 1) / kXcds;
  const int64_t b = blockIdx.x;
  const int64_t u = (b % kXcds) * per + b / kXcds;
  return u < n_units ? u : -1;
}

// Workgroup -> unit for the kernels that write the paged cache (scatter and
// re-rotation). The unit list is walked layer-major (all pages of layer 0,
// then layer 1, ...) and each XCD takes one contiguous eighth of it, so each
// XCD writes the (destination-ordered) pages of a few layers in sequence
// instead of interleaving 32 layer regions. Measured in-process against the
// page-major order: -1.6% scatter and -1.8% re-rotation time at the
// Llama-3-8B shapes. Returns the page-major unit index (page * n_layers +
// layer), or -1 past the end.
__device__ __forceinline__ int64_t layer_major_of(int64_t v, int64_t n_units, int n_layers) {
  const int64_t n_pages = n_units / n_layers;
  const int64_t l = v / n_pages;
  return (v - l * n_pages) * n_layers + l;
}
__device__ __forceinline__ int64_t layer_major_unit(int64_t n_units, int n_layers) {
  const int64_t v = xcd_unit(n_units);
  return v < 0 ? -1 : layer_major_of(v, n_units, n_layers);
}

// Resolves the cache-side and record-side addresses of unit (page, layer),
// page-major. Returns false when the unit's block id or record range is out
// of bounds (the unit is then skipped, never touched).
__device__ __forceinline__ bool unit_addresses(const UnitArgs& a, int64_t unit,
                                               uint8_t** cache, uint8_t** rec,
                                               int* layer) {
  const int64_t p = unit / a.n_layers;
  const int l = (int)(unit - p * a.n_layers);
  const int64_t blk = a.page_ids[p];
  const int64_t off = a.slot_offsets[p] + (int64_t)(a.layer0 + l) * a.layer_bytes;
  if (blk < 0 || blk >= a.num_blocks) return false;
  if (off < 0 || off + 2 * a.page_bytes > a.staging_bytes) return false;
  *cache = reinterpret_cast<uint8_t*>(a.layer_base[l]) + blk * a.page_stride;
  *rec = a.staging + off;
  *layer = l;
  return true;
}

typedef __amdgpu_buffer_rsrc_t rsrc_t;

// A buffer descriptor over [p, p + bytes): out-of-range accesses through it
// read 0 / are dropped by the hardware.
__device__ __forceinline__ rsrc_t make_rsrc(const uint8_t* p, int64_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint8_t*>(p), 0, (int)bytes,
                                           kRsrcWord3);
}
__device__ __forceinline__ u32x4 bload(rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b128(r, off, 0, kLoadPolicy);
}
__device__ __forceinline__ void bstore(rsrc_t r, int off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kStorePolicy);
}

// Copies the two page_bytes runs src_k -> dst_k and src_v -> dst_v, issuing
// all 2*U loads of a round before its stores.
template <int U>
__device__ __forceinline__ void copy_halves(const uint8_t* src_k, const uint8_t* src_v,
                                            uint8_t* dst_k, uint8_t* dst_v,
                                            int64_t page_bytes) {
  const rsrc_t sk = make_rsrc(src_k, page_bytes), sv = make_rsrc(src_v, page_bytes);
  const rsrc_t dk = make_rsrc(dst_k, page_bytes), dv = make_rsrc(dst_v, page_bytes);
  const int nvec = (int)(page_bytes >> 4);
  for (int base = threadIdx.x; base < nvec; base += kThreads * U) {
    u32x4 rk[U], rv[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + k * kThreads;
      if (i < nvec) {
        rk[k] = bload(sk, i << 4);
        rv[k] = bload(sv, i << 4);
      }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + k * kThreads;
      if (i < nvec) {
        bstore(dk, i << 4, rk[k]);
        bstore(dv, i << 4, rv[k]);
      }
    }
  }
}

// Gather: one workgroup per (page, layer) unit, XCD-contiguous order.
__global__ __launch_bounds__(kThreads) void kv_gather_kernel(UnitArgs a) {
  const int64_t u = xcd_unit(a.n_units);
  uint8_t *cache, *rec;
  int l;
  if (u < 0 || !unit_addresses(a, u, &cache, &rec, &l)) return;
  copy_halves<kGatherUnroll>(cache, cache + a.kv_stride, rec, rec + a.page_bytes,
                             a.page_bytes);
}

// Scatter: one workgroup per unit, layer-major per XCD (the host orders the
// page list by destination block, which keeps each layer's page writes
// near-sequential).
__global__ __launch_bounds__(kThreads) void kv_scatter_kernel(UnitArgs a) {
  uint8_t *cache, *rec;
  int l;
  const int64_t u = layer_major_unit(a.n_units, a.n_layers);
  if (u < 0 || !unit_addresses(a, u, &cache, &rec, &l)) return;
  copy_halves<kScatterUnroll>(rec, rec + a.page_bytes, cache, cache + a.kv_stride,
                              a.page_bytes);
}

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

struct RotArgs {
  UnitArgs u;
  const float2* cos_sin;
  const int32_t* rope_idx;
  int32_t n_tables;
  int32_t row_vecs;    // 16-byte vectors per K row (head_dim * e / 16)
  int32_t rot_half;    // rot_dim / 2 (pairs per row)
  int32_t task_vecs;   // rotation tasks per row
  int32_t tail_vec0;   // first un-rotated vector of a row
  int32_t tasks_per_row;
  int32_t rot_vecs;   // 16-byte vectors of a row inside the rotated region
  int32_t half_vecs;  // neox: vectors from a first-half vector to its partner
  const float* k_scale;
};

// Rotates the K page (rows of head_dim elements) from src into dst.
// neox task c: vector c of the first half and its partner at +rot_half;
// gptj task c: vector c, whose VE/2 adjacent pairs rotate in place;
// tail task: one un-rotated 16-byte vector, copied.
// K-page rotation in rounds of kRotUnroll tasks per lane. Task t covers row
// t / tasks_per_row, column c = t % tasks_per_row:
//   neox, c < task_vecs: vector c of the rotated first half and its partner
//                        at +rot_half elements;
//   gptj, c < task_vecs: vector c, whose VE/2 adjacent pairs rotate in place;
//   c >= task_vecs:      one un-rotated 16-byte tail vector, copied.
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
        c_of[k] = c;
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
    constexpr bool kScaled = DT == DSR_DTYPE_FP8_E4M3;
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
  const int64_t u = layer_major_unit(ra.u.n_units, ra.u.n_layers);
  if (u < 0 || !unit_addresses(ra.u, u, &cache, &rec, &l)) return;
  const int64_t p = u / ra.u.n_layers;
  const int ti = ra.rope_idx[p];
  const int64_t pb = ra.u.page_bytes;
  if (ti < 0 || ti >= ra.n_tables) {
    copy_halves<kRotCopyUnroll>(rec, rec + pb, cache, cache + ra.u.kv_stride, pb);
    return;
  }
  const rsrc_t ks = make_rsrc(rec, pb), kd = make_rsrc(cache, pb);
  const rsrc_t vs = make_rsrc(rec + pb, pb), vd = make_rsrc(cache + ra.u.kv_stride, pb);
  const int nvec = (int)(pb >> 4);
  const int row_bytes = ra.row_vecs << 4;
  const int ntask = (int)(pb / row_bytes) * ra.tasks_per_row;
  const int half_off = ra.rot_half * 16 / Codec<DT>::VE;

  VRound<kScatterUnroll> v;
  KRound<DT, STYLE> k;
  v.load(vs, threadIdx.x, nvec);
  k.load(ra, ks, threadIdx.x, ntask, row_bytes, half_off);

  const float2* src_tab = ra.cos_sin + (int64_t)ti * ra.rot_half;
  for (int j = threadIdx.x; j < ra.rot_half; j += kThreads) tab[j] = src_tab[j];
  float scale = 1.0f, inv_scale = 1.0f;
  if (DT == DSR_DTYPE_FP8_E4M3) {
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
  constexpr bool kScaled = DT == DSR_DTYPE_FP8_E4M3;
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
template <int DT, int STYLE, int U>
__device__ __forceinline__ void rotate_contig_round(const RotArgs& ra, VRound<U>& kk,
                                                    int base, int nvec, rsrc_t kd,
                                                    const float2* tab, float scale,
                                                    float inv_scale) {
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int i = base + k * kThreads;
    u32x4 q = kk.r[k];
    if (STYLE == DSR_ROPE_NEOX) {  // whole wave takes part in the shuffle
#pragma unroll
      for (int w = 0; w < 4; ++w) q[w] = (unsigned)__shfl_xor((int)kk.r[k][w], ra.half_vecs);
    }
    if (i >= nvec) continue;
    bstore(kd, i << 4, rotate_vec<DT, STYLE>(ra, kk.r[k], q, i % ra.row_vecs, tab, scale,
                                             inv_scale));
  }
}

// K and V vectors per lane per round: one round covers a 32 KiB bf16 or a
// 16 KiB e4m3 Llama page.
template <int DT>
constexpr int rot_contig_unroll() {
  return DT == DSR_DTYPE_FP8_E4M3 ? 4 : 8;
}

template <int DT, int STYLE>
__global__ __launch_bounds__(kThreads) void kv_scatter_rerotate_contig_kernel(RotArgs ra) {
  __shared__ float2 tab[kMaxRotHalf];
  uint8_t *cache, *rec;
  int l;
  const int64_t u = layer_major_unit(ra.u.n_units, ra.u.n_layers);
  if (u < 0 || !unit_addresses(ra.u, u, &cache, &rec, &l)) return;
  const int64_t p = u / ra.u.n_layers;
  const int ti = ra.rope_idx[p];
  const int64_t pb = ra.u.page_bytes;
  if (ti < 0 || ti >= ra.n_tables) {
    copy_halves<kRotCopyUnroll>(rec, rec + pb, cache, cache + ra.u.kv_stride, pb);
    return;
  }
  constexpr int U = rot_contig_unroll<DT>();
  const rsrc_t ks = make_rsrc(rec, pb), kd = make_rsrc(cache, pb);
  const rsrc_t vs = make_rsrc(rec + pb, pb), vd = make_rsrc(cache + ra.u.kv_stride, pb);
  const int nvec = (int)(pb >> 4);
  VRound<U> v, kk;
  v.load(vs, threadIdx.x, nvec);
  kk.load(ks, threadIdx.x, nvec);
  const float2* src_tab = ra.cos_sin + (int64_t)ti * ra.rot_half;
  for (int j = threadIdx.x; j < ra.rot_half; j += kThreads) tab[j] = src_tab[j];
  float scale = 1.0f, inv_scale = 1.0f;
  if (DT == DSR_DTYPE_FP8_E4M3) {
    scale = ra.k_scale[ra.u.layer0 + l];
    inv_scale = 1.0f / scale;
  }
  __syncthreads();
  const int rounds = (nvec + kThreads * U - 1) / (kThreads * U);
  for (int r = 0; r < rounds; ++r) {  // uniform trip count: shuffles stay converged
    const int base = r * kThreads * U + threadIdx.x;
    if (r > 0) {
      v.load(vs, base, nvec);
      kk.load(ks, base, nvec);
    }
    v.store(vd, base, nvec);
    rotate_contig_round<DT, STYLE, U>(ra, kk, base, nvec, kd, tab, scale, inv_scale);
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
  const int64_t u = layer_major_unit(ra.u.n_units, ra.u.n_layers);
  if (u < 0 || !unit_addresses(ra.u, u, &cache, &rec, &l)) return;
  const int64_t p = u / ra.u.n_layers;
  const int ti = ra.rope_idx[p];
  const int64_t pb = ra.u.page_bytes;
  if (ti < 0 || ti >= ra.n_tables) {
    copy_halves<kRotCopyUnroll>(rec, rec + pb, cache, cache + ra.u.kv_stride, pb);
    return;
  }
  const rsrc_t ks = make_rsrc(rec, pb), kd = make_rsrc(cache, pb);
  const rsrc_t vs = make_rsrc(rec + pb, pb), vd = make_rsrc(cache + ra.u.kv_stride, pb);
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
  if (DT == DSR_DTYPE_FP8_E4M3) {
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

// ---------------------------------------------------------------------------
// Small pages: several units per workgroup.
//
// With one unit per workgroup, a page of a single KV head (4 KiB at head_dim
// 128 bf16) gives each lane one 16-byte vector per run, and the workgroup
// ends after one load latency with 8 KiB moved; a 2 KiB page leaves half the
// lanes idle. The chip then holds too few bytes in flight. Measured at the
// Llama-3-70B TP8 share (4 KiB pages): re-rotation 2.44 TB/s and scatter
// 5.04 TB/s with one unit per workgroup, against 6.1 and 6.5 TB/s grouped.
//
// A grouped workgroup takes G consecutive units of the kernel's unit order
// and sees them as one flat run of G * nvec vectors per half, U vectors per
// lane, all loaded before any store. Pages are a multiple of 1 KiB (one
// wave's 64 vectors) that divides 4 KiB (one workgroup's 256) or is a
// multiple of it, so the unit of every wave's 64 vectors is wave-uniform:
// its addresses come from scalar loads and go into buffer descriptors. The
// kernels are branch-free over the U vectors: a vector with no valid unit
// goes through a zero-size descriptor (loads read 0, stores are dropped);
// branches around each vector made the compiler copy the register arrays
// (256 VGPRs, 1 wave per SIMD, for the re-rotation).

// Units per workgroup for the grouped kernels, 1 when the page does not
// qualify or one unit already fills the budget of U vectors per lane. Env
// DSR_UNITS_PER_GROUP caps G (1 turns the grouped kernels off), for
// in-process comparisons.
int units_per_group(int64_t page_bytes, int u_budget, int cap) {
  if (const char* e = getenv("DSR_UNITS_PER_GROUP")) {
    const int c = atoi(e);
    if (c > 0 && c < cap) cap = c;
  }
  const int64_t nvec = page_bytes >> 4;
  if (nvec % kWave) return 1;
  if (nvec % kThreads && kThreads % nvec) return 1;
  const int64_t g = (int64_t)u_budget * kThreads / nvec;
  if (g <= 1) return 1;
  return g < cap ? (int)g : cap;
}

// Unit v of a page-major (layer fastest) or layer-major (page fastest)
// order, from the position (p0, l0) of the group's first unit: j steps on.
template <bool kPageMajor>
__device__ __forceinline__ void unit_at(const UnitArgs& a, int64_t n_pages, int64_t p0, int l0,
                                        int j, int64_t* p, int* l) {
  if (kPageMajor) {
    int ll = l0 + j;
    int64_t pp = p0;
    while (ll >= a.n_layers) {
      ll -= a.n_layers;
      ++pp;
    }
    *p = pp;
    *l = ll;
  } else {
    int64_t pp = p0 + j;
    int ll = l0;
    while (pp >= n_pages) {
      pp -= n_pages;
      ++ll;
    }
    *p = pp;
    *l = ll;
  }
}

// Descriptors of one unit's cache page and record: size 0 (every access
// dropped) when j is past the group's end or the unit is out of bounds.
struct UnitRsrc {
  const uint8_t* cache;
  const uint8_t* rec;
  int64_t n;
  int64_t p;
  int l;
};

template <bool kPageMajor>
__device__ __forceinline__ UnitRsrc unit_rsrc(const UnitArgs& a, int64_t n_pages, int64_t p0,
                                              int l0, int j, int64_t n_here) {
  UnitRsrc r;
  unit_at<kPageMajor>(a, n_pages, p0, l0, j, &r.p, &r.l);
  bool ok = j < n_here;
  int64_t blk = 0, off = 0;
  if (ok) {
    blk = a.page_ids[r.p];
    off = a.slot_offsets[r.p] + (int64_t)(a.layer0 + r.l) * a.layer_bytes;
    ok = blk >= 0 && blk < a.num_blocks && off >= 0 && off + 2 * a.page_bytes <= a.staging_bytes;
  }
  r.n = ok ? a.page_bytes : 0;
  r.rec = a.staging + (ok ? off : 0);
  r.cache = reinterpret_cast<const uint8_t*>(a.layer_base[ok ? r.l : 0]) +
            (ok ? blk : 0) * a.page_stride;
  if (!ok) r.l = 0;
  return r;
}

// The group of workgroup g: its first unit's (page, layer) and its size.
template <bool kPageMajor>
__device__ __forceinline__ int64_t group_start(const UnitArgs& a, int64_t g, int G,
                                               int64_t n_pages, int64_t* p0, int* l0) {
  const int64_t v0 = g * G;
  if (kPageMajor) {
    *p0 = v0 / a.n_layers;
    *l0 = (int)(v0 - *p0 * a.n_layers);
  } else {
    *l0 = (int)(v0 / n_pages);
    *p0 = v0 - (int64_t)*l0 * n_pages;
  }
  return a.n_units - v0 < G ? a.n_units - v0 : G;
}

// Gather (kGather: page-major, cache -> records) or scatter (layer-major,
// records -> cache) over G units per workgroup.
template <bool kGather, int U>
__global__ __launch_bounds__(kThreads) void kv_copy_grouped_kernel(UnitArgs a, int G) {
  const int64_t g = xcd_unit((a.n_units + G - 1) / G);
  if (g < 0) return;
  const int64_t n_pages = a.n_units / a.n_layers;
  const int nvec = (int)(a.page_bytes >> 4);
  int64_t p0;
  int l0;
  const int64_t n_here = group_start<kGather>(a, g, G, n_pages, &p0, &l0);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int lane = (int)threadIdx.x % kWave;
  u32x4 rk[U], rv[U];
  rsrc_t dk[U], dv[U];
  int off[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int fw = k * kThreads + wave * kWave;  // first flat vector of this wave
    const int j = fw / nvec;
    off[k] = (fw - j * nvec + lane) << 4;
    const UnitRsrc u = unit_rsrc<kGather>(a, n_pages, p0, l0, j, n_here);
    const uint8_t* src = kGather ? u.cache : u.rec;
    const uint8_t* src_v = kGather ? u.cache + a.kv_stride : u.rec + a.page_bytes;
    const uint8_t* dst = kGather ? u.rec : u.cache;
    const uint8_t* dst_v = kGather ? u.rec + a.page_bytes : u.cache + a.kv_stride;
    rk[k] = bload(make_rsrc(src, u.n), off[k]);
    rv[k] = bload(make_rsrc(src_v, u.n), off[k]);
    dk[k] = make_rsrc(dst, u.n);
    dv[k] = make_rsrc(dst_v, u.n);
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    bstore(dk[k], off[k], rk[k]);
    bstore(dv[k], off[k], rv[k]);
  }
}

// Re-rotation over G units per workgroup (layer-major order, as the one-unit
// kernel). The group's (cos, sin) tables are staged in LDS, one rot_half
// stretch per unit; G * rot_half <= kMaxRotHalf. K of an un-rotated unit is
// stored as loaded.
template <int DT, int STYLE>
__global__ __launch_bounds__(kThreads) void kv_scatter_rerotate_grouped_kernel(RotArgs ra,
                                                                               int G) {
  constexpr int U = rot_contig_unroll<DT>();
  __shared__ float2 tab[kMaxRotHalf];
  const UnitArgs& a = ra.u;
  const int64_t g = xcd_unit((a.n_units + G - 1) / G);
  if (g < 0) return;
  const int64_t n_pages = a.n_units / a.n_layers;
  const int nvec = (int)(a.page_bytes >> 4);
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
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int fw = k * kThreads + wave * kWave;
    const int j = fw / nvec;
    off[k] = (fw - j * nvec + lane) << 4;
    const UnitRsrc u = unit_rsrc<false>(a, n_pages, p0, l0, j, n_here);
    rk[k] = bload(make_rsrc(u.rec, u.n), off[k]);
    rv[k] = bload(make_rsrc(u.rec + a.page_bytes, u.n), off[k]);
    kd[k] = make_rsrc(u.cache, u.n);
    vd[k] = make_rsrc(u.cache + a.kv_stride, u.n);
    const int ti = u.n ? ra.rope_idx[u.p] : -1;
    tj[k] = ti >= 0 && ti < ra.n_tables ? j : -1;
    sc[k] = DT == DSR_DTYPE_FP8_E4M3 && u.n ? ra.k_scale[a.layer0 + u.l] : 1.0f;
  }
  // tables of the group's units, fetched while the page loads are in flight
  for (int e = threadIdx.x; e < (int)n_here * ra.rot_half; e += kThreads) {
    const int jj = e / ra.rot_half;
    const int64_t p = (p0 + jj) % n_pages;
    const int ti = ra.rope_idx[p];
    if (ti >= 0 && ti < ra.n_tables)
      tab[e] = ra.cos_sin[(int64_t)ti * ra.rot_half + (e - jj * ra.rot_half)];
  }
#pragma unroll
  for (int k = 0; k < U; ++k) bstore(vd[k], off[k], rv[k]);
  __syncthreads();
#pragma unroll
  for (int k = 0; k < U; ++k) {
    u32x4 q = rk[k];
    if (STYLE == DSR_ROPE_NEOX) {
#pragma unroll
      for (int x = 0; x < 4; ++x) q[x] = (unsigned)__shfl_xor((int)rk[k][x], ra.half_vecs);
    }
    const int t = tj[k] < 0 ? 0 : tj[k];
    const u32x4 r = rotate_vec<DT, STYLE>(ra, rk[k], q, (off[k] >> 4) % ra.row_vecs,
                                          tab + t * ra.rot_half, sc[k], 1.0f / sc[k]);
    bstore(kd[k], off[k], tj[k] < 0 ? rk[k] : r);
  }
}

// ---------------------------------------------------------------------------
// Token-granular (slot_mapping-driven) gather / scatter.

struct SlotArgs {
  const uint64_t* layer_base;
  int64_t kv_stride;
  int64_t page_stride;
  int64_t page_bytes;
  int64_t num_blocks;
  int64_t row_bytes;
  const int64_t* slot_mapping;
  const int64_t* row_offsets;
  uint8_t* staging;
  int64_t staging_bytes;
  int64_t layer_bytes;
  int32_t n_tokens;
  int32_t n_layers;
  int32_t layer0;
  int32_t block_size;
  int32_t block_shift;  // log2(block_size) when a power of two, else -1
};

constexpr int kTokPerWave = 4;  // tokens whose rows a wave has in flight at once
constexpr int kTokPerWg = kTokPerWave * (kThreads / kWave);
constexpr int kRowUnroll = 2;   // 64-vector slices of a row per round

// One workgroup per (16 consecutive tokens, layer); each wave owns 4 of the
// tokens. Token addresses are wave-uniform (scalar loads of slot_mapping and
// row_offsets); the lanes cover a row's 16-byte vectors, so a wave moves a
// token's whole K and V rows, and 4 tokens' rows are in flight together.
template <bool kGather>
__global__ __launch_bounds__(kThreads) void kv_slots_kernel(SlotArgs a) {
  // the scatter writes the paged cache: layer-major per XCD, as the page
  // scatter (-2.4% in-process); the gather keeps the identity order
  int64_t unit = blockIdx.x;
  if (!kGather) {
    const int64_t nu = ((int64_t)a.n_tokens + kTokPerWg - 1) / kTokPerWg * a.n_layers;
    unit = layer_major_unit(nu, a.n_layers);
    if (unit < 0) return;
  }
  const int64_t tb = unit / a.n_layers;
  const int l = (int)(unit - tb * a.n_layers);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int vpr = (int)(a.row_bytes >> 4);
  rsrc_t ck[kTokPerWave], cv[kTokPerWave], rk[kTokPerWave], rv[kTokPerWave];
  bool ok[kTokPerWave];
#pragma unroll
  for (int j = 0; j < kTokPerWave; ++j) {
    const int64_t t = tb * kTokPerWg + wave * kTokPerWave + j;
    ok[j] = false;
    if (t < a.n_tokens) {
      const int64_t slot = a.slot_mapping[t];
      const int64_t blk = slot >= 0 ? slot / a.block_size : -1;
      const int64_t off = a.row_offsets[t] + (int64_t)(a.layer0 + l) * a.layer_bytes;
      ok[j] = blk >= 0 && blk < a.num_blocks && off >= 0 &&
              off + a.page_bytes + a.row_bytes <= a.staging_bytes;
      if (ok[j]) {
        const uint8_t* row = reinterpret_cast<const uint8_t*>(a.layer_base[l]) +
                             blk * a.page_stride + (slot - blk * a.block_size) * a.row_bytes;
        ck[j] = make_rsrc(row, a.row_bytes);
        cv[j] = make_rsrc(row + a.kv_stride, a.row_bytes);
        rk[j] = make_rsrc(a.staging + off, a.row_bytes);
        rv[j] = make_rsrc(a.staging + off + a.page_bytes, a.row_bytes);
      }
    }
  }
  for (int vb = 0; vb < vpr; vb += kWave * kRowUnroll) {
    u32x4 xk[kTokPerWave][kRowUnroll], xv[kTokPerWave][kRowUnroll];
#pragma unroll
    for (int j = 0; j < kTokPerWave; ++j) {
#pragma unroll
      for (int m = 0; m < kRowUnroll; ++m) {
        const int v = vb + m * kWave + lane;
        if (ok[j] && v < vpr) {
          xk[j][m] = bload(kGather ? ck[j] : rk[j], v << 4);
          xv[j][m] = bload(kGather ? cv[j] : rv[j], v << 4);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < kTokPerWave; ++j) {
#pragma unroll
      for (int m = 0; m < kRowUnroll; ++m) {
        const int v = vb + m * kWave + lane;
        if (ok[j] && v < vpr) {
          bstore(kGather ? rk[j] : ck[j], v << 4, xk[j][m]);
          bstore(kGather ? rv[j] : cv[j], v << 4, xv[j][m]);
        }
      }
    }
  }
}

// Rows of at most 32 vectors (512 B: one KV head at head_dim 128 bf16, or
// two at head_dim 64). The kernel above resolves each token with dependent
// scalar loads and a 64-bit division, and keeps 4 tokens per wave in flight
// with a quarter or half of the lanes active: at one and two KV heads it
// measured 1.9 and 3.5 TB/s, against 6.2 for the page kernels of the same
// caches. Here lane j of a wave resolves the wave's token j (one vector load
// of the tables for all of them, a shift for power-of-two block sizes) and
// the wave reads each token's addresses back with readlane; TPW tokens' rows
// are in flight per wave. Branch-free: an invalid token goes through
// zero-size descriptors and lanes past the row end fall outside the
// descriptor, so their loads read 0 and their stores are dropped. Measured
// 5.3 (one head) and 5.7 TB/s (two heads) for the gather.
template <bool kGather, int TPW>
__global__ __launch_bounds__(kThreads) void kv_slots_small_kernel(SlotArgs a) {
  constexpr int kTokWg = TPW * (kThreads / kWave);
  int64_t unit = blockIdx.x;
  if (!kGather) {
    const int64_t nu = ((int64_t)a.n_tokens + kTokWg - 1) / kTokWg * a.n_layers;
    unit = layer_major_unit(nu, a.n_layers);
    if (unit < 0) return;
  }
  const int64_t tb = unit / a.n_layers;
  const int l = (int)(unit - tb * a.n_layers);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int lane = (int)threadIdx.x % kWave;
  // Lane j < TPW resolves token j of the wave (one vector load of the
  // tables for all of them); the wave then reads each token's addresses
  // from its lane.
  const int64_t t0 = tb * kTokWg + (int64_t)wave * TPW;
  const int64_t t = t0 + lane;
  const bool live = lane < TPW && t < a.n_tokens;
  const int64_t slot = live ? a.slot_mapping[t] : -1;
  const int64_t blk = slot < 0 ? -1 : a.block_shift >= 0 ? slot >> a.block_shift : slot / a.block_size;
  const int64_t in_blk = slot - blk * a.block_size;
  const int64_t off = live ? a.row_offsets[t] + (int64_t)(a.layer0 + l) * a.layer_bytes : -1;
  const bool ok = blk >= 0 && blk < a.num_blocks && off >= 0 &&
                  off + a.page_bytes + a.row_bytes <= a.staging_bytes;
  const uint64_t row = reinterpret_cast<uint64_t>(a.layer_base[l]) +
                       (ok ? blk * a.page_stride + in_blk * a.row_bytes : 0);
  const uint64_t rec = reinterpret_cast<uint64_t>(a.staging) + (ok ? off : 0);
  const int n_lane = ok ? (int)a.row_bytes : 0;
  rsrc_t dk[TPW], dv[TPW];
  u32x4 xk[TPW], xv[TPW];
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    const int n = __builtin_amdgcn_readlane(n_lane, j);
    const uint8_t* rj = reinterpret_cast<const uint8_t*>(
        ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(row >> 32), j) << 32) |
        (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)row, j));
    const uint8_t* cj = reinterpret_cast<const uint8_t*>(
        ((uint64_t)(uint32_t)__builtin_amdgcn_readlane((int)(rec >> 32), j) << 32) |
        (uint32_t)__builtin_amdgcn_readlane((int)(uint32_t)rec, j));
    const rsrc_t ck = make_rsrc(rj, n), cv = make_rsrc(rj + a.kv_stride, n);
    const rsrc_t rk = make_rsrc(cj, n), rv = make_rsrc(cj + a.page_bytes, n);
    xk[j] = bload(kGather ? ck : rk, lane << 4);
    xv[j] = bload(kGather ? cv : rv, lane << 4);
    dk[j] = kGather ? rk : ck;
    dv[j] = kGather ? rv : cv;
  }
#pragma unroll
  for (int j = 0; j < TPW; ++j) {
    bstore(dk[j], lane << 4, xk[j]);
    bstore(dv[j], lane << 4, xv[j]);
  }
}

bool aligned16(int64_t v) { return (v & 15) == 0; }
bool aligned16p(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15) == 0; }

int check_common(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                 int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                 const int32_t* page_ids, const int64_t* slot_offsets,
                 int n_pages, const void* staging, int64_t staging_bytes,
                 int64_t layer_bytes, int layer0) {
  if (n_pages < 0 || n_layers < 0 || layer0 < 0 || num_blocks < 0 ||
      staging_bytes < 0 || page_bytes <= 0)
    return DSR_ERR_ARG;
  if (n_pages == 0 || n_layers == 0) return DSR_OK;
  if (!layer_base || !page_ids || !slot_offsets || !staging) return DSR_ERR_ARG;
  if (layer_bytes < 2 * page_bytes) return DSR_ERR_SHAPE;
  if (page_bytes > 0x7fffffffLL) return DSR_ERR_SHAPE;  // one buffer descriptor per run
  if ((int64_t)n_pages * n_layers > 0x7fffffffLL) return DSR_ERR_ARG;
  if (!aligned16(kv_stride) || !aligned16(page_stride) || !aligned16(page_bytes) ||
      !aligned16(layer_bytes) || !aligned16p(staging))
    return DSR_ERR_ALIGN;
  return DSR_OK;
}

UnitArgs make_unit(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                   int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                   const int32_t* page_ids, const int64_t* slot_offsets,
                   int n_pages, const void* staging, int64_t staging_bytes,
                   int64_t layer_bytes, int layer0) {
  UnitArgs a;
  a.layer_base = layer_base;
  a.kv_stride = kv_stride;
  a.page_stride = page_stride;
  a.page_bytes = page_bytes;
  a.num_blocks = num_blocks;
  a.page_ids = page_ids;
  a.slot_offsets = slot_offsets;
  a.staging = const_cast<uint8_t*>(static_cast<const uint8_t*>(staging));
  a.staging_bytes = staging_bytes;
  a.layer_bytes = layer_bytes;
  a.n_layers = n_layers;
  a.layer0 = layer0;
  a.n_units = (int64_t)n_pages * n_layers;
  return a;
}

// Largest workgroup count of one launch: HIP caps gridDim.x * blockDim.x at
// 2^32 - 1 threads (16.7 M workgroups of 256). Env DSR_MAX_WG_PER_LAUNCH
// lowers it, so that tests can exercise the split.
int64_t max_wg_per_launch() {
  int64_t m = 0xffffffffLL / kThreads / kXcds * kXcds;
  if (const char* e = getenv("DSR_MAX_WG_PER_LAUNCH")) {
    const int64_t v = atoll(e) / kXcds * kXcds;
    if (v >= 2 * kXcds && v < m) m = v;
  }
  return m;
}

// Items (pages or tokens) per launch such that ceil(items * n_layers /
// per_wg), rounded up to the XCD count, stays within max_wg_per_launch();
// per_wg = items' units per workgroup (G pages or a block of tokens).
int64_t items_per_launch(int n_layers, int64_t per_wg) {
  const int64_t wg = max_wg_per_launch() - kXcds;
  const int64_t per = wg * per_wg / n_layers;
  return per > 0 ? per : 0;
}

// Launches over consecutive page ranges of `a` (one launch unless the pages
// exceed max_wg_per_launch()), each range's tables offset to its first
// page; launch(b, grid) enqueues one kernel. Grids are a whole multiple of
// the XCD count so that the XCD remap covers every unit. Returns the first
// launch error.
template <class F>
int launch_page_ranges(const UnitArgs& a, int n_pages, int G, F launch) {
  const int64_t per = items_per_launch(a.n_layers, G);
  if (per <= 0) return DSR_ERR_ARG;
  for (int64_t p0 = 0; p0 < n_pages; p0 += per) {
    const int64_t n = n_pages - p0 < per ? n_pages - p0 : per;
    UnitArgs b = a;
    b.page_ids += p0;
    b.slot_offsets += p0;
    b.n_units = n * a.n_layers;
    const unsigned grid = (unsigned)(((b.n_units + G - 1) / G + kXcds - 1) / kXcds * kXcds);
    launch(b, grid);
    const int rc = (int)hipGetLastError();
    if (rc != 0) return rc;
  }
  return DSR_OK;
}

// Dynamic LDS that limits the re-rotation kernel to kRotWgPerCu workgroups
// per CU on the current device (0 if the capacity cannot be read).
size_t rot_occupancy_lds(int wg_per_cu) {
  int dev = 0, lds = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 0;
  if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
                            dev) != hipSuccess || lds <= 0)
    return 0;
  const int64_t want = (int64_t)lds / wg_per_cu - (int64_t)sizeof(float2) * kMaxRotHalf;
  return want > 0 ? (size_t)want : 0;
}

template <int DT>
int launch_rerotate(const RotArgs& ra, int n_pages, int style, hipStream_t s) {
  const int h = ra.half_vecs;
  int wg = rot_wg_per_cu<DT>();
  if (const char* e = getenv("DSR_ROT_WG_PER_CU")) wg = atoi(e) > 0 ? atoi(e) : wg;
  const bool contig = style == DSR_ROPE_GPTJ ||
                      (h > 0 && h <= 32 && (h & (h - 1)) == 0 && ra.row_vecs % (2 * h) == 0);
  const int G = contig ? units_per_group(ra.u.page_bytes, rot_contig_unroll<DT>(),
                                         kMaxRotHalf / ra.rot_half)
                       : 1;
  // neox rows of <= 64 vectors whatever the partner distance: the row-aligned
  // kernel (env DSR_ROT_KERNEL=pairs keeps the pair-task kernel).
  bool rows_ok = !contig && style == DSR_ROPE_NEOX && ra.row_vecs <= kWave && h > 0 &&
                 2 * h <= ra.row_vecs;
  if (const char* e = getenv("DSR_ROT_KERNEL"))
    if (!strcmp(e, "pairs")) rows_ok = false;
  // The grouped kernel also serves pages of exactly U vectors per lane
  // (G = 1), for 16-bit K. Env DSR_ROT_KERNEL=contig|grouped overrides the
  // choice where both apply, for in-process comparisons.
  const int64_t nvec = ra.u.page_bytes >> 4;
  const bool single = contig && nvec % kThreads == 0 &&
                      nvec == (int64_t)rot_contig_unroll<DT>() * kThreads;
  bool grouped = G > 1 || (single && DT != DSR_DTYPE_FP8_E4M3);
  if (const char* e = getenv("DSR_ROT_KERNEL")) {
    if (!strcmp(e, "contig") && contig) grouped = false;
    if (!strcmp(e, "grouped") && (G > 1 || single)) grouped = true;
  }
  if (grouped) {
    wg = G > 1 ? rot_grouped_wg_per_cu<DT>() : kRotSingleWgPerCu;
    if (const char* e = getenv("DSR_ROT_GROUPED_WG_PER_CU")) wg = atoi(e) > 0 ? atoi(e) : wg;
  }
  const size_t dyn = rot_occupancy_lds(wg);
  return launch_page_ranges(ra.u, n_pages, G, [&](const UnitArgs& b, unsigned grid) {
    RotArgs rb = ra;
    rb.u = b;
    rb.rope_idx = ra.rope_idx + (b.page_ids - ra.u.page_ids);
    if (grouped) {
      if (style == DSR_ROPE_NEOX)
        kv_scatter_rerotate_grouped_kernel<DT, DSR_ROPE_NEOX><<<grid, kThreads, dyn, s>>>(rb, G);
      else
        kv_scatter_rerotate_grouped_kernel<DT, DSR_ROPE_GPTJ><<<grid, kThreads, dyn, s>>>(rb, G);
    } else if (contig) {
      if (style == DSR_ROPE_NEOX)
        kv_scatter_rerotate_contig_kernel<DT, DSR_ROPE_NEOX><<<grid, kThreads, dyn, s>>>(rb);
      else
        kv_scatter_rerotate_contig_kernel<DT, DSR_ROPE_GPTJ><<<grid, kThreads, dyn, s>>>(rb);
    } else if (rows_ok) {
      kv_scatter_rerotate_rows_kernel<DT><<<grid, kThreads, dyn, s>>>(rb);
    } else {
      kv_scatter_rerotate_kernel<DT, DSR_ROPE_NEOX><<<grid, kThreads, dyn, s>>>(rb);
    }
  });
}

}  // namespace

extern "C" {

int dsr_abi_version(void) { return DSR_ABI_VERSION; }

const char* dsr_error_string(int code) {
  switch (code) {
    case DSR_OK:
      return "success";
    case DSR_ERR_ARG:
      return "invalid argument (null pointer, negative count or unknown enum)";
    case DSR_ERR_ALIGN:
      return "pointer, stride or size is not a multiple of 16 bytes";
    case DSR_ERR_SHAPE:
      return "inconsistent page/row/rotation geometry";
    case DSR_ERR_IO:
      return "store file read or write failed (see dsr_ring_last_errno)";
    case DSR_ERR_NOFILE:
      return "store file not found";
    default:
      return code > 0 ? hipGetErrorString((hipError_t)code) : "unknown error";
  }
}

int dsr_gather(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
               int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
               const int32_t* page_ids, const int64_t* slot_offsets,
               int n_pages, void* staging, int64_t staging_bytes,
               int64_t layer_bytes, int layer0, dsr_stream_t stream) {
  int rc = check_common(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                        num_blocks, page_ids, slot_offsets, n_pages, staging,
                        staging_bytes, layer_bytes, layer0);
  if (rc != DSR_OK || n_pages == 0 || n_layers == 0) return rc;
  UnitArgs a = make_unit(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                         num_blocks, page_ids, slot_offsets, n_pages, staging,
                         staging_bytes, layer_bytes, layer0);
  // Grouped only below one workgroup's 4 KiB: from 4 KiB up the one-unit
  // kernel measured faster (6.14 vs 5.57 TB/s at 4 KiB pages; 3-8% at 8, 16
  // and 32 KiB).
  const int G = page_bytes < kThreads * 16 ? units_per_group(page_bytes, kGatherUnroll, kMaxGroup) : 1;
  return launch_page_ranges(a, n_pages, G, [&](const UnitArgs& b, unsigned grid) {
    if (G > 1)
      kv_copy_grouped_kernel<true, kGatherUnroll><<<grid, kThreads, 0, (hipStream_t)stream>>>(b, G);
    else
      kv_gather_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>(b);
  });
}

int dsr_scatter(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                const int32_t* page_ids, const int64_t* slot_offsets,
                int n_pages, const void* staging, int64_t staging_bytes,
                int64_t layer_bytes, int layer0, dsr_stream_t stream) {
  int rc = check_common(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                        num_blocks, page_ids, slot_offsets, n_pages, staging,
                        staging_bytes, layer_bytes, layer0);
  if (rc != DSR_OK || n_pages == 0 || n_layers == 0) return rc;
  UnitArgs a = make_unit(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                         num_blocks, page_ids, slot_offsets, n_pages, staging,
                         staging_bytes, layer_bytes, layer0);
  // Grouped up to 4 KiB pages (6.47 vs 5.04 TB/s at 4 KiB); at 8-32 KiB the
  // one-unit kernel measured equal or faster.
  const int G = page_bytes <= kThreads * 16 ? units_per_group(page_bytes, kScatterUnroll, kMaxGroup) : 1;
  return launch_page_ranges(a, n_pages, G, [&](const UnitArgs& b, unsigned grid) {
    if (G > 1)
      kv_copy_grouped_kernel<false, kScatterUnroll><<<grid, kThreads, 0, (hipStream_t)stream>>>(b, G);
    else
      kv_scatter_kernel<<<grid, kThreads, 0, (hipStream_t)stream>>>(b);
  });
}

int dsr_scatter_rerotate(const uint64_t* layer_base, int n_layers,
                         int64_t kv_stride, int64_t page_stride,
                         int64_t page_bytes, int64_t num_blocks,
                         const int32_t* page_ids, const int64_t* slot_offsets,
                         int n_pages, const void* staging,
                         int64_t staging_bytes, int64_t layer_bytes,
                         int layer0, const float* cos_sin,
                         const int32_t* rope_idx, int n_tables, int head_dim,
                         int rot_dim, int rope_style, int dtype,
                         const float* k_scale, dsr_stream_t stream) {
  int rc = check_common(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                        num_blocks, page_ids, slot_offsets, n_pages, staging,
                        staging_bytes, layer_bytes, layer0);
  if (rc != DSR_OK) return rc;
  if (rope_style != DSR_ROPE_NEOX && rope_style != DSR_ROPE_GPTJ) return DSR_ERR_ARG;
  int esize, ve;
  switch (dtype) {
    case DSR_DTYPE_BF16:
    case DSR_DTYPE_FP16:
      esize = 2;
      ve = 8;
      break;
    case DSR_DTYPE_FP8_E4M3:
      esize = 1;
      ve = 16;
      break;
    default:
      return DSR_ERR_ARG;
  }
  if (n_tables < 0) return DSR_ERR_ARG;
  if (head_dim <= 0 || rot_dim <= 0 || rot_dim > head_dim || (rot_dim & 1) ||
      rot_dim / 2 > kMaxRotHalf)
    return DSR_ERR_SHAPE;
  const int64_t row_bytes = (int64_t)head_dim * esize;
  if (row_bytes % 16 || page_bytes % row_bytes) return DSR_ERR_SHAPE;
  if (((int64_t)(head_dim - rot_dim) * esize) % 16) return DSR_ERR_SHAPE;
  int task_vecs;
  if (rope_style == DSR_ROPE_NEOX) {
    if ((rot_dim / 2) % ve) return DSR_ERR_SHAPE;
    task_vecs = rot_dim / 2 / ve;
  } else {
    if (rot_dim % ve) return DSR_ERR_SHAPE;
    task_vecs = rot_dim / ve;
  }
  if (n_pages == 0 || n_layers == 0) return DSR_OK;
  if (!rope_idx || (n_tables > 0 && !cos_sin)) return DSR_ERR_ARG;
  if (dtype == DSR_DTYPE_FP8_E4M3 && !k_scale) return DSR_ERR_ARG;

  RotArgs ra;
  ra.u = make_unit(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                   num_blocks, page_ids, slot_offsets, n_pages, staging,
                   staging_bytes, layer_bytes, layer0);
  ra.cos_sin = reinterpret_cast<const float2*>(cos_sin);
  ra.rope_idx = rope_idx;
  ra.n_tables = n_tables;
  ra.row_vecs = (int)(row_bytes / 16);
  ra.rot_half = rot_dim / 2;
  ra.task_vecs = task_vecs;
  ra.tail_vec0 = rot_dim * esize / 16;
  ra.tasks_per_row = task_vecs + (head_dim - rot_dim) * esize / 16;
  ra.rot_vecs = rot_dim * esize / 16;
  ra.half_vecs = rope_style == DSR_ROPE_NEOX ? rot_dim / 2 * esize / 16 : 0;
  ra.k_scale = k_scale;
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case DSR_DTYPE_BF16:
      return launch_rerotate<DSR_DTYPE_BF16>(ra, n_pages, rope_style, s);
    case DSR_DTYPE_FP16:
      return launch_rerotate<DSR_DTYPE_FP16>(ra, n_pages, rope_style, s);
    default:
      return launch_rerotate<DSR_DTYPE_FP8_E4M3>(ra, n_pages, rope_style, s);
  }
}

namespace {

int slots_launch(bool gather, const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                 int64_t page_stride, int64_t page_bytes, int64_t num_blocks, int block_size,
                 int64_t row_bytes, const int64_t* slot_mapping, const int64_t* row_offsets,
                 int n_tokens, const void* staging, int64_t staging_bytes,
                 int64_t layer_bytes, int layer0, dsr_stream_t stream) {
  if (n_tokens < 0 || n_layers < 0 || layer0 < 0 || num_blocks < 0 || staging_bytes < 0 ||
      block_size <= 0 || row_bytes <= 0 || page_bytes <= 0)
    return DSR_ERR_ARG;
  if (n_tokens == 0 || n_layers == 0) return DSR_OK;
  if (!layer_base || !slot_mapping || !row_offsets || !staging) return DSR_ERR_ARG;
  if (page_bytes < (int64_t)block_size * row_bytes || layer_bytes < 2 * page_bytes ||
      row_bytes > 0x7fffffffLL)
    return DSR_ERR_SHAPE;
  if (!aligned16(kv_stride) || !aligned16(page_stride) || !aligned16(page_bytes) ||
      !aligned16(row_bytes) || !aligned16(layer_bytes) || !aligned16p(staging))
    return DSR_ERR_ALIGN;
  const int64_t vpr = row_bytes >> 4;
  // Tokens per wave for small rows, measured in-process (ragged requests,
  // 80 layers): 8 at 16-vector rows (4.34 ms gather vs 4.39 at 4 and 16),
  // 4 at 32-vector rows (8.19 ms vs 8.35-8.45). 0: the large-row kernel.
  int tpw = vpr <= 16 ? 8 : vpr <= 32 ? 4 : 0;
  if (const char* e = getenv("DSR_SLOTS_TPW"))  // tuning override for small rows
    if (tpw && (atoi(e) == 4 || atoi(e) == 8 || atoi(e) == 16)) tpw = atoi(e);
  const int tok_wg = tpw ? tpw * (kThreads / kWave) : kTokPerWg;
  const int64_t blocks = ((int64_t)n_tokens + tok_wg - 1) / tok_wg;
  if (blocks * n_layers > 0x7fffffffLL) return DSR_ERR_ARG;
  SlotArgs a;
  a.layer_base = layer_base;
  a.kv_stride = kv_stride;
  a.page_stride = page_stride;
  a.page_bytes = page_bytes;
  a.num_blocks = num_blocks;
  a.row_bytes = row_bytes;
  a.slot_mapping = slot_mapping;
  a.row_offsets = row_offsets;
  a.staging = const_cast<uint8_t*>(static_cast<const uint8_t*>(staging));
  a.staging_bytes = staging_bytes;
  a.layer_bytes = layer_bytes;
  a.n_tokens = n_tokens;
  a.n_layers = n_layers;
  a.layer0 = layer0;
  a.block_size = block_size;
  a.block_shift = (block_size & (block_size - 1)) == 0 ? __builtin_ctz((unsigned)block_size) : -1;
  hipStream_t s = (hipStream_t)stream;
  // token ranges whose launches stay within max_wg_per_launch()
  const int64_t per = items_per_launch(n_layers, tok_wg) / tok_wg * tok_wg;
  if (per <= 0) return DSR_ERR_ARG;
  for (int64_t t0 = 0; t0 < n_tokens; t0 += per) {
    SlotArgs b = a;
    b.slot_mapping += t0;
    b.row_offsets += t0;
    b.n_tokens = (int32_t)(n_tokens - t0 < per ? n_tokens - t0 : per);
    const int64_t units = ((int64_t)b.n_tokens + tok_wg - 1) / tok_wg * n_layers;
    const unsigned grid = (unsigned)(gather ? units : (units + kXcds - 1) / kXcds * kXcds);
    if (tpw == 16) {
      if (gather)
        kv_slots_small_kernel<true, 16><<<grid, kThreads, 0, s>>>(b);
      else
        kv_slots_small_kernel<false, 16><<<grid, kThreads, 0, s>>>(b);
    } else if (tpw == 8) {
      if (gather)
        kv_slots_small_kernel<true, 8><<<grid, kThreads, 0, s>>>(b);
      else
        kv_slots_small_kernel<false, 8><<<grid, kThreads, 0, s>>>(b);
    } else if (tpw == 4) {
      if (gather)
        kv_slots_small_kernel<true, 4><<<grid, kThreads, 0, s>>>(b);
      else
        kv_slots_small_kernel<false, 4><<<grid, kThreads, 0, s>>>(b);
    } else if (gather) {
      kv_slots_kernel<true><<<grid, kThreads, 0, s>>>(b);
    } else {
      kv_slots_kernel<false><<<grid, kThreads, 0, s>>>(b);
    }
    const int rc = (int)hipGetLastError();
    if (rc != 0) return rc;
  }
  return DSR_OK;
}

}  // namespace

int dsr_gather_slots(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                     int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                     int block_size, int64_t row_bytes, const int64_t* slot_mapping,
                     const int64_t* row_offsets, int n_tokens, void* staging,
                     int64_t staging_bytes, int64_t layer_bytes, int layer0,
                     dsr_stream_t stream) {
  return slots_launch(true, layer_base, n_layers, kv_stride, page_stride, page_bytes,
                      num_blocks, block_size, row_bytes, slot_mapping, row_offsets, n_tokens,
                      staging, staging_bytes, layer_bytes, layer0, stream);
}

int dsr_scatter_slots(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                      int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                      int block_size, int64_t row_bytes, const int64_t* slot_mapping,
                      const int64_t* row_offsets, int n_tokens, const void* staging,
                      int64_t staging_bytes, int64_t layer_bytes, int layer0,
                      dsr_stream_t stream) {
  return slots_launch(false, layer_base, n_layers, kv_stride, page_stride, page_bytes,
                      num_blocks, block_size, row_bytes, slot_mapping, row_offsets, n_tokens,
                      staging, staging_bytes, layer_bytes, layer0, stream);
}

}  // extern "C"
