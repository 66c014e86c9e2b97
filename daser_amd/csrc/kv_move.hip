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
// moves it with 16-byte lane vectors (global_load_dwordx4 /
// global_store_dwordx4), issuing every load of a round before any store so
// each lane keeps up to 2*kUnroll 16-byte requests in flight. No LDS is
// needed for the copy: both sides are contiguous within a unit. The
// re-rotation kernel keeps the unit's (cos, sin) table in LDS.
//
// Reference being replaced: the Python per-(request, block, layer) torch
// copy_ loops of daser/connector/daser_connector.py:536-551 (load) and
// :610-632 (save).

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "daser_kv.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));

constexpr int kThreads = 256;   // 4 wave64 per workgroup
constexpr int kCopyUnroll = 8;  // 16-byte vectors per lane per half per round
constexpr int kRotUnroll = 4;   // rotation tasks per lane per round
constexpr int kMaxRotHalf = 512;  // LDS table capacity: rot_dim <= 1024

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
  int32_t n_layers;
  int32_t layer0;
};

// Resolves the cache-side and record-side addresses of the workgroup's unit.
// Returns false when the unit's block id or record range is out of bounds
// (the unit is then skipped, never touched).
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

__device__ __forceinline__ u32x4 ld16(const uint8_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}
__device__ __forceinline__ u32x4 ld16_stream(const uint8_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ void st16(uint8_t* p, u32x4 v) {
  *reinterpret_cast<u32x4*>(p) = v;
}
__device__ __forceinline__ void st16_stream(uint8_t* p, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
}

// Copies the two page_bytes runs (K at +0, V at +kv_src_off / +kv_dst_off).
// Record-side accesses are streamed (non-temporal): records are produced once
// and consumed by a DMA or consumed once by the load.
template <bool kToRecord>
__device__ __forceinline__ void copy_halves(const uint8_t* src_k,
                                            const uint8_t* src_v,
                                            uint8_t* dst_k, uint8_t* dst_v,
                                            int64_t page_bytes) {
  const int64_t nvec = page_bytes >> 4;
  for (int64_t base = threadIdx.x; base < nvec;
       base += (int64_t)kThreads * kCopyUnroll) {
    u32x4 rk[kCopyUnroll], rv[kCopyUnroll];
#pragma unroll
    for (int k = 0; k < kCopyUnroll; ++k) {
      const int64_t i = base + (int64_t)k * kThreads;
      if (i < nvec) {
        if (kToRecord) {
          rk[k] = ld16(src_k + (i << 4));
          rv[k] = ld16(src_v + (i << 4));
        } else {
          rk[k] = ld16_stream(src_k + (i << 4));
          rv[k] = ld16_stream(src_v + (i << 4));
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kCopyUnroll; ++k) {
      const int64_t i = base + (int64_t)k * kThreads;
      if (i < nvec) {
        if (kToRecord) {
          st16_stream(dst_k + (i << 4), rk[k]);
          st16_stream(dst_v + (i << 4), rv[k]);
        } else {
          st16(dst_k + (i << 4), rk[k]);
          st16(dst_v + (i << 4), rv[k]);
        }
      }
    }
  }
}

// One workgroup per (page, layer) unit; grid.x = n_pages * n_layers.
template <bool kGather>
__global__ __launch_bounds__(kThreads) void kv_page_copy_kernel(UnitArgs a) {
  uint8_t *cache, *rec;
  int l;
  if (!unit_addresses(a, blockIdx.x, &cache, &rec, &l)) return;
  if (kGather) {
    copy_halves<true>(cache, cache + a.kv_stride, rec, rec + a.page_bytes,
                      a.page_bytes);
  } else {
    copy_halves<false>(rec, rec + a.page_bytes, cache, cache + a.kv_stride,
                       a.page_bytes);
  }
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

// OCP e4m3fn decode: bias 7, no infinities, S.1111.111 is NaN.
__device__ __forceinline__ float e4m3_to_f32(uint32_t b) {
  const uint32_t sign = (b & 0x80u) << 24;
  const uint32_t em = b & 0x7fu;
  if (em == 0x7fu) return __uint_as_float(0x7fc00000u | sign);
  float mag;
  if (em >= 0x08u) {
    // normal: exponent field e in [1,15] -> fp32 exponent e + 120
    mag = __uint_as_float((em + (120u << 3)) << 20);
  } else {
    mag = (float)em * 0x1p-9f;  // subnormal: m * 2^-9, exact
  }
  return __uint_as_float(__float_as_uint(mag) | sign);
}
// fp32 -> e4m3fn, round-to-nearest-even, |f| saturated to 448 first;
// NaN -> 0x7F.
__device__ __forceinline__ uint32_t f32_to_e4m3(float f) {
  if (__builtin_isnan(f)) return 0x7fu;
  f = f > 448.0f ? 448.0f : (f < -448.0f ? -448.0f : f);
  uint32_t u = __float_as_uint(f);
  const uint32_t sign = (u >> 24) & 0x80u;
  u &= 0x7fffffffu;
  if (u >= 0x3c800000u) {  // |f| >= 2^-6: normal range of e4m3
    u += 0x7ffffu + ((u >> 20) & 1u);
    return sign | ((u - (120u << 23)) >> 20);
  }
  // subnormal range: m = rne(|f| * 2^9) in [0, 8]; 8 encodes 2^-6 exactly
  const float m = __builtin_rintf(__uint_as_float(u) * 512.0f);
  return sign | (uint32_t)m;
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
    for (int k = 0; k < 16; ++k) x[k] = e4m3_to_f32((v[k >> 2] >> (8 * (k & 3))) & 0xffu);
  }
  __device__ static u32x4 encode(const float* y) {
    u32x4 v = {0u, 0u, 0u, 0u};
#pragma unroll
    for (int k = 0; k < 16; ++k) v[k >> 2] |= f32_to_e4m3(y[k]) << (8 * (k & 3));
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
  const float* k_scale;
};

// Rotates the K page (rows of head_dim elements) from src into dst.
// neox task c: vector c of the first half and its partner at +rot_half;
// gptj task c: vector c, whose VE/2 adjacent pairs rotate in place;
// tail task: one un-rotated 16-byte vector, copied.
template <int DT, int STYLE>
__device__ __forceinline__ void rotate_k_page(const RotArgs& ra,
                                              const uint8_t* src, uint8_t* dst,
                                              const float2* tab, float scale,
                                              float inv_scale) {
  using C = Codec<DT>;
  constexpr int VE = C::VE;
  const int64_t row_bytes = (int64_t)ra.row_vecs << 4;
  const int64_t rows = ra.u.page_bytes / row_bytes;
  const int64_t ntask = rows * ra.tasks_per_row;
  const int64_t half_off = (int64_t)ra.rot_half * 16 / VE;  // bytes to partner
  for (int64_t base = threadIdx.x; base < ntask;
       base += (int64_t)kThreads * kRotUnroll) {
    u32x4 a[kRotUnroll], b[kRotUnroll];
    int64_t off[kRotUnroll];
    int kind[kRotUnroll];  // 0 = rotate, 1 = copy, -1 = none
    int c_of[kRotUnroll];
#pragma unroll
    for (int k = 0; k < kRotUnroll; ++k) {
      const int64_t t = base + (int64_t)k * kThreads;
      kind[k] = -1;
      if (t < ntask) {
        const int64_t row = t / ra.tasks_per_row;
        const int c = (int)(t - row * ra.tasks_per_row);
        c_of[k] = c;
        if (c < ra.task_vecs) {
          kind[k] = 0;
          off[k] = row * row_bytes + ((int64_t)c << 4);
          a[k] = ld16_stream(src + off[k]);
          if (STYLE == DSR_ROPE_NEOX) b[k] = ld16_stream(src + off[k] + half_off);
        } else {
          kind[k] = 1;
          off[k] = row * row_bytes + ((int64_t)(ra.tail_vec0 + c - ra.task_vecs) << 4);
          a[k] = ld16_stream(src + off[k]);
        }
      }
    }
#pragma unroll
    for (int k = 0; k < kRotUnroll; ++k) {
      if (kind[k] == 1) {
        st16(dst + off[k], a[k]);
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
            const float x1 = x[e] * scale, x2 = z[e] * scale;
            x[e] = (x1 * cs.x - x2 * cs.y) * inv_scale;
            z[e] = (x2 * cs.x + x1 * cs.y) * inv_scale;
          }
          st16(dst + off[k], C::encode(x));
          st16(dst + off[k] + half_off, C::encode(z));
        } else {
          const int j0 = c_of[k] * (VE / 2);
#pragma unroll
          for (int e = 0; e < VE / 2; ++e) {
            const float2 cs = tab[j0 + e];
            const float x1 = x[2 * e] * scale, x2 = x[2 * e + 1] * scale;
            x[2 * e] = (x1 * cs.x - x2 * cs.y) * inv_scale;
            x[2 * e + 1] = (x2 * cs.x + x1 * cs.y) * inv_scale;
          }
          st16(dst + off[k], C::encode(x));
        }
      }
    }
  }
}

template <int DT, int STYLE>
__global__ __launch_bounds__(kThreads) void kv_scatter_rerotate_kernel(RotArgs ra) {
  __shared__ float2 tab[kMaxRotHalf];
  uint8_t *cache, *rec;
  int l;
  if (!unit_addresses(ra.u, blockIdx.x, &cache, &rec, &l)) return;
  const int64_t p = (int64_t)blockIdx.x / ra.u.n_layers;
  const int ti = ra.rope_idx[p];
  const int64_t pb = ra.u.page_bytes;
  // V half (and K when not rotated) is a plain copy.
  if (ti < 0 || ti >= ra.n_tables) {
    copy_halves<false>(rec, rec + pb, cache, cache + ra.u.kv_stride, pb);
    return;
  }
  const float2* src_tab = ra.cos_sin + (int64_t)ti * ra.rot_half;
  for (int j = threadIdx.x; j < ra.rot_half; j += kThreads) tab[j] = src_tab[j];
  float scale = 1.0f, inv_scale = 1.0f;
  if (DT == DSR_DTYPE_FP8_E4M3) {
    scale = ra.k_scale[ra.u.layer0 + l];
    inv_scale = 1.0f / scale;
  }
  __syncthreads();
  // V: copy with the full unroll (no rotation).
  {
    const uint8_t* sv = rec + pb;
    uint8_t* dv = cache + ra.u.kv_stride;
    const int64_t nvec = pb >> 4;
    for (int64_t base = threadIdx.x; base < nvec;
         base += (int64_t)kThreads * kCopyUnroll) {
      u32x4 r[kCopyUnroll];
#pragma unroll
      for (int k = 0; k < kCopyUnroll; ++k) {
        const int64_t i = base + (int64_t)k * kThreads;
        if (i < nvec) r[k] = ld16_stream(sv + (i << 4));
      }
#pragma unroll
      for (int k = 0; k < kCopyUnroll; ++k) {
        const int64_t i = base + (int64_t)k * kThreads;
        if (i < nvec) st16(dv + (i << 4), r[k]);
      }
    }
  }
  rotate_k_page<DT, STYLE>(ra, rec, cache, tab, scale, inv_scale);
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
  if ((int64_t)n_pages * n_layers > 0x7fffffffLL) return DSR_ERR_ARG;
  if (!aligned16(kv_stride) || !aligned16(page_stride) || !aligned16(page_bytes) ||
      !aligned16(layer_bytes) || !aligned16p(staging))
    return DSR_ERR_ALIGN;
  return DSR_OK;
}

UnitArgs make_unit(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                   int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                   const int32_t* page_ids, const int64_t* slot_offsets,
                   const void* staging, int64_t staging_bytes,
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
  return a;
}

template <int DT>
int launch_rerotate(const RotArgs& ra, int style, unsigned grid, hipStream_t s) {
  if (style == DSR_ROPE_NEOX)
    kv_scatter_rerotate_kernel<DT, DSR_ROPE_NEOX><<<grid, kThreads, 0, s>>>(ra);
  else
    kv_scatter_rerotate_kernel<DT, DSR_ROPE_GPTJ><<<grid, kThreads, 0, s>>>(ra);
  return (int)hipGetLastError();
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
                         num_blocks, page_ids, slot_offsets, staging,
                         staging_bytes, layer_bytes, layer0);
  const unsigned grid = (unsigned)((int64_t)n_pages * n_layers);
  kv_page_copy_kernel<true><<<grid, kThreads, 0, (hipStream_t)stream>>>(a);
  return (int)hipGetLastError();
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
                         num_blocks, page_ids, slot_offsets, staging,
                         staging_bytes, layer_bytes, layer0);
  const unsigned grid = (unsigned)((int64_t)n_pages * n_layers);
  kv_page_copy_kernel<false><<<grid, kThreads, 0, (hipStream_t)stream>>>(a);
  return (int)hipGetLastError();
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
                   num_blocks, page_ids, slot_offsets, staging, staging_bytes,
                   layer_bytes, layer0);
  ra.cos_sin = reinterpret_cast<const float2*>(cos_sin);
  ra.rope_idx = rope_idx;
  ra.n_tables = n_tables;
  ra.row_vecs = (int)(row_bytes / 16);
  ra.rot_half = rot_dim / 2;
  ra.task_vecs = task_vecs;
  ra.tail_vec0 = rot_dim * esize / 16;
  ra.tasks_per_row = task_vecs + (head_dim - rot_dim) * esize / 16;
  ra.k_scale = k_scale;
  const unsigned grid = (unsigned)((int64_t)n_pages * n_layers);
  hipStream_t s = (hipStream_t)stream;
  switch (dtype) {
    case DSR_DTYPE_BF16:
      return launch_rerotate<DSR_DTYPE_BF16>(ra, rope_style, grid, s);
    case DSR_DTYPE_FP16:
      return launch_rerotate<DSR_DTYPE_FP16>(ra, rope_style, grid, s);
    default:
      return launch_rerotate<DSR_DTYPE_FP8_E4M3>(ra, rope_style, grid, s);
  }
}

}  // extern "C"
