// kv_page_kernels.h -- page gather and scatter, one unit per workgroup and grouped
// (several units per workgroup for small pages).
// Part of libdaser_kv: included by kv_move.hip, one translation unit.

#pragma once

#include "kv_common.h"

namespace {

// Gather: one workgroup per (page, layer) unit, XCD-contiguous order. The
// kSplit instance has a.parts consecutive workgroups share a unit, each
// copying its part of both runs; it is a separate instance because the
// split arithmetic cost 1.7% at 4 KiB pages.
template <bool kSplit>
__global__ __launch_bounds__(kThreads) void kv_gather_kernel(UnitArgs a) {
  const int64_t w = xcd_unit(kSplit ? a.n_units * a.parts : a.n_units);
  if (w < 0) return;
  const int64_t u = kSplit ? udiv32(w, a.parts) : w;
  const int64_t bytes = kSplit ? a.page_bytes / a.parts : a.page_bytes;
  const int64_t part = kSplit ? bytes * (w - u * a.parts) : 0;
  uint8_t *cache, *rec;
  int l;
  if (!unit_addresses(a, u, &cache, &rec, &l)) return;
  copy_halves<kGatherUnroll>(cache + part, cache + a.kv_stride + part, rec + part,
                             rec + a.page_bytes + part, bytes);
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

// Scatter of pages of 32 KiB and up (larger ones in 32 KiB parts),
// launched at one workgroup per CU (the launch policy keeps about 64 KiB of
// each CU's units in flight; see copy_wg_per_cu in kv_move.hip). Each lane keeps U (8 at 32 KiB)
// vectors of K and of V in flight, and every store follows its own load's
// arrival (no wait for the whole round): at one workgroup per CU the waves
// stream instead of alternating a load burst with a store burst. Measured
// in-process at the Llama-3-8B shape (32 KiB pages) on three boxes: 12.27 vs
// 12.60 ms, 11.98 vs 12.08, 11.97 vs 12.09 for kv_scatter_kernel at its
// register-limited 3 workgroups per CU; kv_scatter_kernel itself at one
// workgroup per CU 12.54-12.56 ms. Units in hardware dispatch order
// (kHwOrder): a further 3.5%. Pages above 32 KiB go as 32 KiB parts, one
// workgroup each (kSplit): a workgroup's second round waits for its first
// round's stores (vmcnt counts both), and parts measured 13% faster at 64
// KiB pages (Llama-3-8B with block_size 32: 5.10 vs 5.75 ms). U = 4 serves 16 KiB
// pages (e4m3) for measurements: at two workgroups per CU it measured
// 23.0-23.6 ms at config 4 in three processes on one box against
// 21.8-24.0 ms for kv_scatter_kernel, the spread being the buffers'
// placement, so the default stays kv_scatter_kernel there.
template <int U, bool kHwOrder, bool kSplit = false>
__global__ __launch_bounds__(kThreads) void kv_scatter_stream_kernel(UnitArgs a) {
  uint8_t *cache, *rec;
  int l;
  // kSplit: a.parts consecutive workgroups share a unit (pages above 32
  // KiB: one round of U vectors per lane each), as consecutive units of the
  // same order
  const int64_t nw = kSplit ? a.n_units * a.parts : a.n_units;
  const int64_t b = kHwOrder ? ((int64_t)blockIdx.x < nw ? (int64_t)blockIdx.x : -1)
                             : xcd_unit(nw);
  if (b < 0) return;
  const int64_t v = kSplit ? udiv32(b, a.parts) : b;
  const int64_t u = layer_major_of(v, a.n_units, a.n_layers);
  if (!unit_addresses(a, u, &cache, &rec, &l)) return;
  const int64_t pb = kSplit ? a.page_bytes / a.parts : a.page_bytes;
  const int64_t part = kSplit ? pb * (b - v * a.parts) : 0;
  const rsrc_t sk = make_rsrc(rec + part, pb), sv = make_rsrc(rec + a.page_bytes + part, pb);
  const rsrc_t dk = make_rsrc(cache + part, pb), dv = make_rsrc(cache + a.kv_stride + part, pb);
  const int nvec = (int)(pb >> 4);
  for (int base = threadIdx.x; base < nvec; base += kThreads * U) {
    u32x4 xk[U], xv[U];
#pragma unroll
    for (int k = 0; k < U; ++k) {
      xk[k] = bload(sk, (base + k * kThreads) << 4);
      xv[k] = bload(sv, (base + k * kThreads) << 4);
    }
#pragma unroll
    for (int k = 0; k < U; ++k) {
      bstore(dk, (base + k * kThreads) << 4, xk[k]);
      bstore(dv, (base + k * kThreads) << 4, xv[k]);
    }
  }
}

// Gather and scatter of head-major cache pages (records in token-major
// order), one unit per workgroup, in the unit orders above.
template <bool kGather>
__global__ __launch_bounds__(kThreads) void kv_copy_hnd_kernel(UnitArgs a) {
  uint8_t *cache, *rec;
  int l;
  const int64_t u = kGather ? xcd_unit(a.n_units) : layer_major_unit(a.n_units, a.n_layers);
  if (u < 0 || !unit_addresses(a, u, &cache, &rec, &l)) return;
  copy_halves_hnd<kHndUnroll, kGather>(a, cache, rec);
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
// qualify or one unit already fills the budget of U vectors per lane. The
// DSR_TUNE_UNITS_PER_GROUP override caps G (1 turns the grouped kernels off), for
// in-process comparisons.
int units_per_group(int64_t page_bytes, int u_budget, int cap) {
  if (const int64_t c = tune(DSR_TUNE_UNITS_PER_GROUP)) {
    if (c > 0 && c < cap) cap = (int)c;
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
    *p0 = udiv32(v0, a.n_layers);
    *l0 = (int)(v0 - *p0 * a.n_layers);
  } else {
    *l0 = (int)udiv32(v0, n_pages);
    *p0 = v0 - (int64_t)*l0 * n_pages;
  }
  return a.n_units - v0 < G ? a.n_units - v0 : G;
}

// Gather (kGather: page-major, cache -> records) or scatter (layer-major,
// records -> cache) over G units per workgroup. HND: head-major cache pages
// (the cache side of each vector goes through hnd_vec).
template <bool kGather, int U, bool HND = false>
__global__ __launch_bounds__(kThreads) void kv_copy_grouped_kernel(UnitArgs a, int G) {
  const int64_t g = xcd_unit(udiv32(a.n_units + G - 1, G));
  if (g < 0) return;
  const int64_t n_pages = udiv32(a.n_units, a.n_layers);
  const int nvec = (int)(a.page_bytes >> 4);
  int64_t p0;
  int l0;
  const int64_t n_here = group_start<kGather>(a, g, G, n_pages, &p0, &l0);
  const int wave = __builtin_amdgcn_readfirstlane((int)threadIdx.x / kWave);
  const int lane = (int)threadIdx.x % kWave;
  u32x4 rk[U], rv[U];
  rsrc_t dk[U], dv[U];
  int off[U], doff[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    const int fw = k * kThreads + wave * kWave;  // first flat vector of this wave
    const int j = fw / nvec;
    off[k] = (fw - j * nvec + lane) << 4;
    const int coff = HND ? hnd_vec(a, off[k] >> 4) << 4 : off[k];  // cache side
    const UnitRsrc u = unit_rsrc<kGather>(a, n_pages, p0, l0, j, n_here);
    const uint8_t* src = kGather ? u.cache : u.rec;
    const uint8_t* src_v = kGather ? u.cache + a.kv_stride : u.rec + a.page_bytes;
    const uint8_t* dst = kGather ? u.rec : u.cache;
    const uint8_t* dst_v = kGather ? u.rec + a.page_bytes : u.cache + a.kv_stride;
    rk[k] = bload(make_rsrc(src, u.n), kGather ? coff : off[k]);
    rv[k] = bload(make_rsrc(src_v, u.n), kGather ? coff : off[k]);
    dk[k] = make_rsrc(dst, u.n);
    dv[k] = make_rsrc(dst_v, u.n);
    doff[k] = kGather ? off[k] : coff;
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    bstore(dk[k], doff[k], rk[k]);
    bstore(dv[k], doff[k], rv[k]);
  }
}

}  // namespace
