// kv_common.h -- constants, cache policies, the (page, layer) unit and its orders,
// buffer descriptors and the copy engine shared by the kernels.
// Part of libdaser_kv: included by kv_move.hip, one translation unit.

#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <atomic>

#include "daser_kv.h"

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef unsigned int u32x2 __attribute__((ext_vector_type(2)));

constexpr int kThreads = 256;     // 4 wave64 per workgroup
constexpr int kWave = 64;
constexpr int kMaxGroup = 64;     // units per workgroup of the grouped copy kernels
constexpr int kGatherUnroll = 16;  // 16-byte vectors per lane per half per round
constexpr int kScatterUnroll = 16;
constexpr int kRotCopyUnroll = 8;  // copy of unrotated pages inside the re-rotation kernels
constexpr int kHndUnroll = 8;      // head-major page copies
constexpr int kRotUnroll = 4;      // rotation tasks per lane per round (pair-task kernel)
constexpr int kMaxRotHalf = 512;   // LDS table capacity: rot_dim <= 1024
constexpr int kXcds = 8;           // MI355X: 8 XCDs, workgroups dealt round-robin

// Cache-policy bits of gfx950 buffer instructions (CPol: sc0 = 1, nt = 2,
// sc1 = 16). Loads stream through (nt); stores are written with sc0 sc1,
// which measured fastest for these write-once streams (6.0 vs 5.2 TB/s for
// default-policy stores at the Llama-3-8B shape).
constexpr int kLoadPolicy = 2;
constexpr int kStorePolicy = 17;
// Launch-shape overrides for measurements and tests, set through
// dsr_set_tuning() (0 = the geometry's own choice). Nothing reads the
// environment: a serving process gets the defaults unless its code asks.
// Relaxed atomics, read once per call.
enum RotKernelOverride { kRotAuto = 0, kRotPairs = 1, kRotContig = 2, kRotGrouped = 3 };
struct TuningKnobs {
  std::atomic<int64_t> v[DSR_TUNE_COUNT_];
};
TuningKnobs g_tuning{};
inline int64_t tune(int knob) { return g_tuning.v[knob].load(std::memory_order_relaxed); }

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
  // Head-major cache pages ([H][block_size][row] in memory while records
  // hold [block_size][H][row]): rows of hnd_row_vecs vectors; 0 = pages in
  // record order.
  int32_t hnd_heads = 0;
  int32_t hnd_block = 0;
  int32_t hnd_row_vecs = 0;
  // Workgroups per unit of the one-unit gather and streaming scatter (1, or
  // a count whose share of the page is a whole number of 4 KiB blocks):
  // pages above 32 KiB, and launches with too few units to fill the chip,
  // split each unit's two runs into equal parts.
  int32_t parts = 1;
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
// Unit, page and token counts of one launch stay below 2^31 (the entry
// points check), so the index arithmetic divides in 32 bits: a 64-bit
// division is a long instruction sequence, paid by every workgroup.
__device__ __forceinline__ int64_t udiv32(int64_t x, int64_t d) {
  return (int64_t)((uint32_t)x / (uint32_t)d);
}
__device__ __forceinline__ int64_t layer_major_of(int64_t v, int64_t n_units, int n_layers) {
  const uint32_t n_pages = (uint32_t)n_units / (uint32_t)n_layers;
  const uint32_t l = (uint32_t)v / n_pages;
  return (int64_t)((uint32_t)v - l * n_pages) * n_layers + l;
}
__device__ __forceinline__ int64_t layer_major_unit(int64_t n_units, int n_layers) {
  const int64_t v = xcd_unit(n_units);
  return v < 0 ? -1 : layer_major_of(v, n_units, n_layers);
}

// The same layer-major walk in hardware dispatch order: consecutive
// workgroups (dealt round-robin to the 8 XCDs) take consecutive units, so at
// any moment the whole chip works on one stretch of one layer's
// destination-ordered pages. Used by the streaming scatter at one workgroup
// per CU: 256 adjacent pages in flight write one K and one V window of
// 8 MiB each, against 8 XCDs x 2 windows in the XCD-contiguous order.
// Measured in-process: 11.87 vs 12.29 ms at config 2 and 6.70 vs 6.97 ms
// at config 3's pages; the kernels at three workgroups per CU, the
// re-rotations and the e4m3 (16 KiB) pages ran 1-14% slower in this order.
__device__ __forceinline__ int64_t layer_major_unit_hw(int64_t n_units, int n_layers) {
  const int64_t b = blockIdx.x;
  return b < n_units ? layer_major_of(b, n_units, n_layers) : -1;
}

// Resolves the cache-side and record-side addresses of unit (page, layer),
// page-major. Returns false when the unit's block id or record range is out
// of bounds (the unit is then skipped, never touched).
__device__ __forceinline__ bool unit_addresses(const UnitArgs& a, int64_t unit,
                                               uint8_t** cache, uint8_t** rec,
                                               int* layer) {
  const uint32_t p = (uint32_t)unit / (uint32_t)a.n_layers;
  const int l = (int)((uint32_t)unit - p * (uint32_t)a.n_layers);
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
// 8-byte load with the default (cached) policy, for small shared tables
__device__ __forceinline__ u32x2 bload_b64(rsrc_t r, int off) {
  return __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, 0);
}
__device__ __forceinline__ void bstore(rsrc_t r, int off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kStorePolicy);
}

// Head-major pages: record vector i (row r = t * H + h of token t, head h)
// is cache vector (h * block_size + t) * row_vecs + its column.
__device__ __forceinline__ int hnd_vec(const UnitArgs& a, int i) {
  const int r = i / a.hnd_row_vecs, v = i - r * a.hnd_row_vecs;
  const int t = r / a.hnd_heads, h = r - t * a.hnd_heads;
  return (h * a.hnd_block + t) * a.hnd_row_vecs + v;
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

// copy_halves between a head-major cache page and its record: the record
// side is walked lane-consecutively, the cache side through hnd_vec (whole
// rows stay contiguous, so a row's lanes still coalesce). Vectors past the
// page are skipped, as in copy_halves (issuing them against an empty range
// cost 40% at 4 KiB pages).
template <int U, bool kGather>
__device__ __forceinline__ void copy_halves_hnd(const UnitArgs& a, uint8_t* cache,
                                                uint8_t* rec) {
  const int64_t pb = a.page_bytes;
  const rsrc_t ck = make_rsrc(cache, pb), cv = make_rsrc(cache + a.kv_stride, pb);
  const rsrc_t rk = make_rsrc(rec, pb), rv = make_rsrc(rec + pb, pb);
  const int nvec = (int)(pb >> 4);
  for (int base = threadIdx.x; base < nvec; base += kThreads * U) {
    u32x4 xk[U], xv[U];
    int ro[U], co[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + k * kThreads;
      if (i < nvec) {
        ro[k] = i << 4;
        co[k] = hnd_vec(a, i) << 4;
        xk[k] = bload(kGather ? ck : rk, kGather ? co[k] : ro[k]);
        xv[k] = bload(kGather ? cv : rv, kGather ? co[k] : ro[k]);
      }
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      const int i = base + k * kThreads;
      if (i < nvec) {
        bstore(kGather ? rk : ck, kGather ? ro[k] : co[k], xk[k]);
        bstore(kGather ? rv : cv, kGather ? ro[k] : co[k], xv[k]);
      }
    }
  }
}

}  // namespace
