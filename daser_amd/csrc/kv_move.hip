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
//     (kv_copy_grouped_kernel); pages above 32 KiB take one workgroup per
//     32 KiB part, and gathers of few units split their units further.
//   re-rotation: kv_scatter_rerotate_grouped_kernel for pages below U * 4
//     KiB and 16-bit pages of exactly U * 4 KiB (and 16-bit token-major pages
//     of several such parts, one workgroup each); kv_scatter_rerotate_contig_
//     kernel for other larger pages with a power-of-two partner distance;
//     kv_scatter_rerotate_rows_kernel for other neox rows of <= 64 vectors;
//     the pair-task kv_scatter_rerotate_kernel otherwise; rotary widths that
//     are not whole 16-byte vectors: kv_scatter_rerotate_lds_kernel.
//   token form (dsr_gather_slots / dsr_scatter_slots): kv_slots_packed_kernel
//     for power-of-two rows of <= 8 vectors, kv_slots_small_kernel for other
//     rows of <= 32 vectors, kv_slots_kernel above.
//   split-x K pages (dsr_scatter_rerotate_kx): the contig and grouped
//     kernels with the KX flag, or the pair-task kernel.
//   head-major cache pages (dsr_*_hnd): the same kernels as token-major
//     pages of that size with the HND flag (kv_copy_hnd_kernel for one unit
//     per workgroup), whose cache-side offsets go through hnd_vec.
// Calls too large for one launch run as several over page (token) ranges.
//
// Reference being replaced: the Python per-(request, block, layer) torch
// copy_ loops of daser/connector/daser_connector.py:536-551 (load) and
// :610-632 (save).

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include <mutex>

#include "daser_kv.h"

#include "kv_common.h"
#include "kv_page_kernels.h"
#include "kv_rotate.h"
#include "kv_slots.h"
#include "kv_fanout.h"

namespace {

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
  UnitArgs a{};
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
// 2^32 - 1 threads (16.7 M workgroups of 256). The DSR_TUNE_MAX_WG_PER_LAUNCH
// override lowers it, so that tests can exercise the split.
int64_t max_wg_per_launch() {
  int64_t m = 0xffffffffLL / kThreads / kXcds * kXcds;
  if (const int64_t t = tune(DSR_TUNE_MAX_WG_PER_LAUNCH)) {
    const int64_t v = t / kXcds * kXcds;
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
  // a.parts workgroups per unit (the split kernels) count as a.parts units
  const int64_t per = items_per_launch(a.n_layers * a.parts, G);
  if (per <= 0) return DSR_ERR_ARG;
  for (int64_t p0 = 0; p0 < n_pages; p0 += per) {
    const int64_t n = n_pages - p0 < per ? n_pages - p0 : per;
    UnitArgs b = a;
    b.page_ids += p0;
    b.slot_offsets += p0;
    b.n_units = n * a.n_layers;
    const unsigned grid =
        (unsigned)(((b.n_units * a.parts + G - 1) / G + kXcds - 1) / kXcds * kXcds);
    launch(b, grid);
    const int rc = (int)hipGetLastError();
    if (rc != 0) return rc;
  }
  return DSR_OK;
}

// Workgroups per CU for the re-rotation kernel, applied with dynamic LDS
// sized from the CU's LDS capacity (the DSR_TUNE_ROT_WG_PER_CU override changes it, for
// tuning). Measured in-process at the Llama-3-8B shapes: 16-bit K (64 KiB
// per unit) runs best at 2-3 per CU (7.67 ms vs 7.87 ms at 4-8 and 11.0 ms
// at 1); e4m3 (32 KiB per unit) at 4 per CU (24.17 ms; 24.4-24.5 ms at 6-12,
// 30.1 ms at 2).
template <int DT>
constexpr int rot_wg_per_cu() {
  return is_fp8<DT>() ? 4 : 2;
}
// The same for the grouped re-rotation kernel (pages below U * 4 KiB; env
// DSR_ROT_GROUPED_WG_PER_CU overrides). Measured in-process at the
// Llama-3-70B TP8 share: 16-bit K 6.97 ms at 4 per CU (7.41 at 2, 7.07 at
// 8); e4m3 with 2 KiB pages 3.24 ms at 8 per CU (3.56 at 4), with 8 KiB
// pages 12.96 ms at 8 (13.72 at 4).
template <int DT>
constexpr int rot_grouped_wg_per_cu() {
  return is_fp8<DT>() ? 8 : 4;
}
// The grouped kernel with one unit per workgroup (16-bit pages of exactly
// U * 4 KiB, the Llama-3-8B/70B shapes): 3 per CU. Measured in-process:
// config 3 7.05 ms at 2-3 per CU, 7.36 at 4-5 (the contig kernel 7.68);
// config 5 55.1 ms at 2-3, 50.4 at 4-6 (contig 55.4), where the shared
// source chunks' reads hit the memory-side cache. 3 is taken for the
// HBM-bound case, 4 when the caller flags shared records
// (DSR_REROTATE_SHARED_RECORDS). e4m3 keeps the contig kernel (24.05 vs
// 24.22 ms at config 4).
constexpr int kRotSingleWgPerCu = 3;
constexpr int kRotSingleSharedWgPerCu = 4;
// Dynamic LDS that limits a kernel with `static_lds` bytes of static LDS to
// wg_per_cu workgroups per CU on the current device (0 if the capacity cannot
// be read). The capacity is read once per device.
constexpr int64_t kLdsGranule = 512;
constexpr int kMaxDevices = 64;
std::atomic<int> g_lds_per_cu[kMaxDevices];
size_t occupancy_lds(int wg_per_cu, int64_t static_lds) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || wg_per_cu <= 0) return 0;
  int lds = dev < kMaxDevices ? g_lds_per_cu[dev].load(std::memory_order_relaxed) : 0;
  if (lds <= 0) {
    if (hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor,
                              dev) != hipSuccess || lds <= 0)
      return 0;
    if (dev < kMaxDevices) g_lds_per_cu[dev].store(lds, std::memory_order_relaxed);
  }
  // a workgroup's LDS (static plus dynamic) is allocated in 512-byte
  // granules: round its share down so that wg_per_cu of them fit
  const int64_t share = (int64_t)lds / wg_per_cu / kLdsGranule * kLdsGranule;
  const int64_t want = share - static_lds;
  return want > 0 ? (size_t)want : 0;
}
size_t rot_occupancy_lds(int wg_per_cu) {
  return occupancy_lds(wg_per_cu, (int64_t)sizeof(float2) * kMaxRotHalf);
}

// Workgroups per CU for the one-unit page copies (0: no limit; the copy
// kernels' registers allow 3). Units in flight per CU are limited to about
// 64 KiB of pages (K + V): one workgroup per CU at 32 KiB pages, two at 16
// KiB. Measured in-process (ms, 3 per CU -> this policy): Llama-3-8B bf16
// (32 KiB pages) scatter 12.08 -> 11.97 (stream kernel), gather 11.75 ->
// 11.60, on three boxes alike; e4m3 (16 KiB pages) scatter 24.71 -> 24.07,
// gather 22.07 -> 22.09. More than 64 KiB in flight per CU makes the DRAM
// side slower, not faster (fewer, longer-waiting requests win); one
// workgroup per CU at 16 KiB pages leaves the CU idle between units (28.4 ms).
// Launches of fewer than kPacedMinUnits units (a single layer's save of a
// step, ...) keep the registers' three workgroups per CU, with dynamic LDS
// sized for three (one layer's scatter of 1,024-4,096 pages: 23.1 vs 24.4
// and 83.4 vs 86.0 us without LDS; gathers alike): they end before a steady
// state, and one per CU measured 0-11% slower there (one layer, 1,024-4,096
// pages: gather 21.8 vs 19.6 us, 99 vs 94 us), against 1% faster from 8,192
// units.
constexpr int64_t kPacedMinUnits = 8192;
int copy_wg_per_cu(int64_t page_bytes, int64_t n_units) {
  if (const int64_t t = tune(DSR_TUNE_COPY_WG_PER_CU)) return (int)t;
  if (n_units < kPacedMinUnits) return 3;
  const int64_t w = (64 << 10) / (2 * page_bytes);
  return w >= 3 ? 0 : (int)(w < 1 ? 1 : w);
}

// Workgroups per unit of a one-unit gather launch (a layer's save of a
// serving step moves 16-4,096 pages). Few units leave most CUs idle; split
// units finish sooner. A part stays a whole number of 4 KiB (one vector per
// lane). Measured per launch at the Llama-3-8B shape (32 KiB pages, rocprofv3
// kernel durations, medians of 128 launches; split 1 -> chosen): 16 pages
// 4.32 -> 3.32 us (8), 64 pages 5.36 -> 4.32 (8), 128 pages 6.16 -> 5.68
// (4; 8: 6.52), 512 pages 14.5-15.2 -> 13.8 (2), 1,024 pages 26.9-27.5 ->
// 25.0 (2), 2,048 pages 49.5 -> 46.9 (2), 4,096 pages 93.3 -> 90.8 (2); at
// 256 pages (7.7-7.8 vs 7.9-8.2) and from 6,144 pages (equal, 4 slower)
// one workgroup per unit stays. The DSR_TUNE_GATHER_SPLIT override sets it
// (1: off).
int gather_split(int64_t page_bytes, int64_t n_units) {
  int64_t s = tune(DSR_TUNE_GATHER_SPLIT);
  if (!s)
    s = n_units <= 64 ? 8 : n_units <= 128 ? 4 : n_units >= 512 && n_units <= 4096 ? 2 : 1;
  while (s > 1 && (page_bytes % (s * kThreads * 16) != 0 || n_units * s > max_wg_per_launch()))
    s /= 2;
  return (int)(s < 1 ? 1 : s);
}

// Parts of a page above 32 KiB for the one-unit gather and the streaming
// scatter: 32 KiB each (the copies' tuned unit; a workgroup's later rounds
// would wait for its earlier stores, since vmcnt counts both). The
// DSR_TUNE_PAGE_PARTS override sets it (1: whole pages).
constexpr int64_t kPartBytes = 32 << 10;
int page_parts(int64_t page_bytes) {
  if (const int64_t t = tune(DSR_TUNE_PAGE_PARTS))
    return page_bytes % (t * kThreads * 16) == 0 ? (int)t : 1;
  return page_bytes > kPartBytes && page_bytes % kPartBytes == 0 ? (int)(page_bytes / kPartBytes)
                                                                 : 1;
}

template <int DT>
int launch_rerotate(const RotArgs& ra, int n_pages, int style, bool vec_ok, hipStream_t s,
                    bool kx, unsigned flags, bool hnd = false) {
  const int h = ra.half_vecs;
  int wg = rot_wg_per_cu<DT>();
  if (const int64_t t = tune(DSR_TUNE_ROT_WG_PER_CU)) wg = t > 0 ? (int)t : wg;
  const int64_t rot_kernel = tune(DSR_TUNE_ROT_KERNEL);
  if (!vec_ok) {  // rotary width not in whole vectors: the LDS kernel
    return launch_page_ranges(ra.u, n_pages, 1, [&](const UnitArgs& b, unsigned grid) {
      RotArgs rb = ra;
      rb.u = b;
      rb.rope_idx = ra.rope_idx + (b.page_ids - ra.u.page_ids);
      if (style == DSR_ROPE_NEOX)
        kv_scatter_rerotate_lds_kernel<DT, DSR_ROPE_NEOX><<<grid, kThreads, 0, s>>>(rb);
      else
        kv_scatter_rerotate_lds_kernel<DT, DSR_ROPE_GPTJ><<<grid, kThreads, 0, s>>>(rb);
    });
  }
  // split-x K (kx): the caller checked the kx_phys conditions, which make
  // every neox partner lane ^ 32
  const bool contig = kx || hnd || style == DSR_ROPE_GPTJ ||
                      (h > 0 && h <= 32 && (h & (h - 1)) == 0 && ra.row_vecs % (2 * h) == 0);
  const int G = contig ? units_per_group(ra.u.page_bytes, rot_contig_unroll<DT>(),
                                         kMaxRotHalf / ra.rot_half)
                       : 1;
  // neox rows of <= 64 vectors whatever the partner distance: the row-aligned
  // kernel (the DSR_TUNE_ROT_KERNEL override "pairs" keeps the pair-task kernel).
  bool rows_ok = !contig && style == DSR_ROPE_NEOX && ra.row_vecs <= kWave && h > 0 &&
                 2 * h <= ra.row_vecs;
  if (rot_kernel == kRotPairs) rows_ok = false;
  // The grouped kernel also serves pages of exactly U vectors per lane
  // (G = 1), for 16-bit K. The DSR_TUNE_ROT_KERNEL override (contig, grouped) changes the
  // choice where both apply, for in-process comparisons.
  // 16-bit token-major pages above 32 KiB run the grouped kernel's single-
  // unit path on 32 KiB parts, one workgroup each (the DSR_TUNE_PAGE_PARTS
  // override 1 keeps whole pages on the contig kernel)
  const int64_t part_vecs = (int64_t)rot_contig_unroll<DT>() * kThreads;
  const int64_t row_bytes = (int64_t)ra.row_vecs * 16;
  int parts = 1;
  if (contig && !kx && !hnd && !is_fp8<DT>() && tune(DSR_TUNE_PAGE_PARTS) != 1 &&
      (ra.u.page_bytes >> 4) > part_vecs && (ra.u.page_bytes >> 4) % part_vecs == 0 &&
      (part_vecs * 16) % row_bytes == 0)
    parts = (int)((ra.u.page_bytes >> 4) / part_vecs);
  const int64_t nvec = (ra.u.page_bytes >> 4) / parts;
  const bool single = contig && nvec % kThreads == 0 && nvec == part_vecs;
  bool grouped = G > 1 || (single && !is_fp8<DT>());
  if (rot_kernel == kRotContig && contig && parts == 1) grouped = false;
  if (rot_kernel == kRotGrouped && (G > 1 || single)) grouped = true;
  if (grouped) {
    wg = G > 1 ? rot_grouped_wg_per_cu<DT>()
         : (flags & DSR_REROTATE_SHARED_RECORDS) ? kRotSingleSharedWgPerCu
                                                 : kRotSingleWgPerCu;
    if (const int64_t t = tune(DSR_TUNE_ROT_GROUPED_WG_PER_CU)) wg = t > 0 ? (int)t : wg;
  }
  const size_t dyn = rot_occupancy_lds(wg);
  // units per workgroup of the kernel actually launched: the one-unit
  // kernels (an override may pick contig where G > 1) take one
  const int GL = grouped ? G : 1;
  UnitArgs ua = ra.u;
  ua.parts = grouped ? parts : 1;
  if (!grouped && !contig && rows_ok) {
    // the row-aligned kernel on large pages: parts of whole rows near 32 KiB
    const int64_t pbytes = ra.u.page_bytes;
    int best = 1;
    if (const int64_t t = tune(DSR_TUNE_PAGE_PARTS)) {
      if (pbytes % t == 0 && (pbytes / t) % row_bytes == 0) best = (int)t;
    } else if (pbytes > kPartBytes) {
      int64_t bd = pbytes - kPartBytes;
      for (int q = 2; q <= 8; ++q) {
        const int64_t pt = pbytes / q;
        if (pbytes % q || pt % row_bytes || pt < (16 << 10)) continue;
        const int64_t d = pt > kPartBytes ? pt - kPartBytes : kPartBytes - pt;
        if (d < bd) bd = d, best = q;
      }
    }
    ua.parts = best;
  }
  return launch_page_ranges(ua, n_pages, GL, [&](const UnitArgs& b, unsigned grid) {
    RotArgs rb = ra;
    rb.u = b;
    // one unit per workgroup over distinct records: the whole chip on one
    // stretch of one layer, as the streaming scatter (config 3: 6.89-6.92 vs
    // 7.04-7.05 ms on two boxes); several units per workgroup (8.1% slower
    // at the TP8 share) and shared records (equal) keep the XCD order
    rb.hw_order = grouped && GL == 1 && !(flags & DSR_SHARED_RECORDS);
    rb.rope_idx = ra.rope_idx + (b.page_ids - ra.u.page_ids);
    if (grouped) {
      if (hnd && style == DSR_ROPE_NEOX)
        kv_scatter_rerotate_grouped_kernel<DT, DSR_ROPE_NEOX, false, true><<<grid, kThreads, dyn, s>>>(rb, GL);
      else if (hnd)
        kv_scatter_rerotate_grouped_kernel<DT, DSR_ROPE_GPTJ, false, true><<<grid, kThreads, dyn, s>>>(rb, GL);
      else if (style == DSR_ROPE_NEOX && kx)
        kv_scatter_rerotate_grouped_kernel<DT, DSR_ROPE_NEOX, true><<<grid, kThreads, dyn, s>>>(rb, GL);
      else if (style == DSR_ROPE_NEOX)
        kv_scatter_rerotate_grouped_kernel<DT, DSR_ROPE_NEOX, false><<<grid, kThreads, dyn, s>>>(rb, GL);
      else if (kx)
        kv_scatter_rerotate_grouped_kernel<DT, DSR_ROPE_GPTJ, true><<<grid, kThreads, dyn, s>>>(rb, GL);
      else
        kv_scatter_rerotate_grouped_kernel<DT, DSR_ROPE_GPTJ, false><<<grid, kThreads, dyn, s>>>(rb, GL);
    } else if (contig) {
      if (hnd && style == DSR_ROPE_NEOX)
        kv_scatter_rerotate_contig_kernel<DT, DSR_ROPE_NEOX, false, true><<<grid, kThreads, dyn, s>>>(rb);
      else if (hnd)
        kv_scatter_rerotate_contig_kernel<DT, DSR_ROPE_GPTJ, false, true><<<grid, kThreads, dyn, s>>>(rb);
      else if (style == DSR_ROPE_NEOX && kx)
        kv_scatter_rerotate_contig_kernel<DT, DSR_ROPE_NEOX, true><<<grid, kThreads, dyn, s>>>(rb);
      else if (style == DSR_ROPE_NEOX)
        kv_scatter_rerotate_contig_kernel<DT, DSR_ROPE_NEOX, false><<<grid, kThreads, dyn, s>>>(rb);
      else if (kx)
        kv_scatter_rerotate_contig_kernel<DT, DSR_ROPE_GPTJ, true><<<grid, kThreads, dyn, s>>>(rb);
      else
        kv_scatter_rerotate_contig_kernel<DT, DSR_ROPE_GPTJ, false><<<grid, kThreads, dyn, s>>>(rb);
    } else if (rows_ok) {
      kv_scatter_rerotate_rows_kernel<DT><<<grid, kThreads, dyn, s>>>(rb);
    } else {
      kv_scatter_rerotate_kernel<DT, DSR_ROPE_NEOX><<<grid, kThreads, dyn, s>>>(rb);
    }
  });
}

// The pair-task kernel alone: the split-x K layout, whose rotation partners
// are a whole block of vectors apart.
template <int DT>
int launch_rerotate_pairs(const RotArgs& ra, int n_pages, int style, hipStream_t s) {
  const size_t dyn = rot_occupancy_lds(rot_wg_per_cu<DT>());
  return launch_page_ranges(ra.u, n_pages, 1, [&](const UnitArgs& b, unsigned grid) {
    RotArgs rb = ra;
    rb.u = b;
    rb.rope_idx = ra.rope_idx + (b.page_ids - ra.u.page_ids);
    if (style == DSR_ROPE_NEOX)
      kv_scatter_rerotate_kernel<DT, DSR_ROPE_NEOX><<<grid, kThreads, dyn, s>>>(rb);
    else
      kv_scatter_rerotate_kernel<DT, DSR_ROPE_GPTJ><<<grid, kThreads, dyn, s>>>(rb);
  });
}

}  // namespace

extern "C" {

int dsr_abi_version(void) { return DSR_ABI_VERSION; }

int dsr_set_tuning(int knob, int64_t value) {
  if (knob < 0 || knob >= DSR_TUNE_COUNT_ || value < 0) return DSR_ERR_ARG;
  g_tuning.v[knob].store(value, std::memory_order_relaxed);
  return DSR_OK;
}

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
    case DSR_ERR_TOO_LARGE:
      return "tables exceed the library's static table area (DSR_STATIC_TABLE_BYTES)";
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
  int split = 1;
  if (G == 1) {
    const int pp = page_parts(page_bytes);
    split = gather_split(page_bytes / pp, a.n_units * pp);
    a.parts = pp * split;
  }
  return launch_page_ranges(a, n_pages, G, [&](const UnitArgs& b, unsigned grid) {
    const hipStream_t st = (hipStream_t)stream;
    if (G > 1) {
      kv_copy_grouped_kernel<true, kGatherUnroll><<<grid, kThreads, 0, st>>>(b, G);
    } else {
      // launches split for lack of units keep the registers' three
      // workgroups per CU (they end before a steady state)
      const int64_t wus = b.n_units * b.parts;  // workgroup-sized units
      const size_t dyn =
          occupancy_lds(split > 1 ? 3 : copy_wg_per_cu(page_bytes / b.parts, wus), 0);
      if (b.parts > 1)
        kv_gather_kernel<true><<<grid, kThreads, dyn, st>>>(b);
      else
        kv_gather_kernel<false><<<grid, kThreads, dyn, st>>>(b);
    }
  });
}

int dsr_scatter_ex(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                   int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                   const int32_t* page_ids, const int64_t* slot_offsets,
                   int n_pages, const void* staging, int64_t staging_bytes,
                   int64_t layer_bytes, int layer0, unsigned flags, dsr_stream_t stream) {
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
  // records read by several pages are partly served by the caches, so
  // more bytes in flight pay (the 70B share's 64 shared chunks: 50.5 ms at
  // the registers' 3 workgroups per CU vs 52.6 ms at one)
  const bool shared = (flags & DSR_SHARED_RECORDS) && !tune(DSR_TUNE_COPY_WG_PER_CU);
  // the streaming kernel moves pages above 32 KiB as 32 KiB parts, one
  // workgroup each; U vectors per lane per round (8 for multiples of 32 KiB,
  // 4 for 16 KiB multiples)
  const int pp = G == 1 && !shared ? page_parts(page_bytes) : 1;
  const int64_t part_bytes = page_bytes / pp;
  const int su = part_bytes % (kThreads * 8 * 16) == 0 ? 8
                 : part_bytes % (kThreads * 4 * 16) == 0 ? 4 : 0;
  const int64_t pick = tune(DSR_TUNE_SCATTER_KERNEL);
  const int wpc_part = shared ? 0 : copy_wg_per_cu(part_bytes, a.n_units * pp);
  const int64_t kind = pick ? pick : wpc_part == 1 && su == 8 ? 2 : 1;
  const bool stream_k = G == 1 && (kind == 2 || kind == 3) && su != 0;
  if (stream_k) a.parts = pp;
  const int wpc = stream_k ? wpc_part : shared ? 0 : copy_wg_per_cu(page_bytes, a.n_units);
  return launch_page_ranges(a, n_pages, G, [&](const UnitArgs& b, unsigned grid) {
    const hipStream_t st = (hipStream_t)stream;
    if (G > 1) {
      // dynamic LDS for the registers' three workgroups per CU: 6.95 vs
      // 7.10 ms at the 70B TP8 share's 4 KiB pages (the same effect as for
      // the token kernels; the gather measured alike with and without)
      kv_copy_grouped_kernel<false, kScatterUnroll><<<grid, kThreads, occupancy_lds(3, 0), st>>>(b, G);
      return;
    }
    const size_t dyn = occupancy_lds(wpc, 0);
    const bool hw = kind == 2, split = b.parts > 1;
    if (!stream_k)
      kv_scatter_kernel<<<grid, kThreads, dyn, st>>>(b);
    else if (su == 8 && hw && split)
      kv_scatter_stream_kernel<8, true, true><<<grid, kThreads, dyn, st>>>(b);
    else if (su == 8 && hw)
      kv_scatter_stream_kernel<8, true><<<grid, kThreads, dyn, st>>>(b);
    else if (su == 8 && split)
      kv_scatter_stream_kernel<8, false, true><<<grid, kThreads, dyn, st>>>(b);
    else if (su == 8)
      kv_scatter_stream_kernel<8, false><<<grid, kThreads, dyn, st>>>(b);
    else if (hw && split)
      kv_scatter_stream_kernel<4, true, true><<<grid, kThreads, dyn, st>>>(b);
    else if (hw)
      kv_scatter_stream_kernel<4, true><<<grid, kThreads, dyn, st>>>(b);
    else if (split)
      kv_scatter_stream_kernel<4, false, true><<<grid, kThreads, dyn, st>>>(b);
    else
      kv_scatter_stream_kernel<4, false><<<grid, kThreads, dyn, st>>>(b);
  });
}

int dsr_scatter(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                const int32_t* page_ids, const int64_t* slot_offsets,
                int n_pages, const void* staging, int64_t staging_bytes,
                int64_t layer_bytes, int layer0, dsr_stream_t stream) {
  return dsr_scatter_ex(layer_base, n_layers, kv_stride, page_stride, page_bytes, num_blocks,
                        page_ids, slot_offsets, n_pages, staging, staging_bytes, layer_bytes,
                        layer0, 0u, stream);
}

}  // extern "C"

namespace {

// All K layouts: kx_block = 0 for token-major K rows (block_size x H x D),
// kx_block = block_size for the split-x K layout (H x D/X x block_size x X);
// hnd_block = block_size for head-major cache pages (H x block_size x D,
// records token-major).
int scatter_rerotate_any(const uint64_t* layer_base, int n_layers,
                         int64_t kv_stride, int64_t page_stride,
                         int64_t page_bytes, int64_t num_blocks,
                         const int32_t* page_ids, const int64_t* slot_offsets,
                         int n_pages, const void* staging,
                         int64_t staging_bytes, int64_t layer_bytes,
                         int layer0, const float* cos_sin,
                         const int32_t* rope_idx, int n_tables,
                         const int32_t* layer_group, int n_groups, int head_dim,
                         int rot_dim, int rope_style, int dtype,
                         const float* k_scale, int kx_block, int hnd_block, unsigned flags,
                         dsr_stream_t stream) {
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
    case DSR_DTYPE_FP8_E5M2:
      esize = 1;
      ve = 16;
      break;
    default:
      return DSR_ERR_ARG;
  }
  if (n_tables < 0 || (layer_group && n_groups < 1)) return DSR_ERR_ARG;
  if (head_dim <= 0 || rot_dim <= 0 || rot_dim > head_dim || (rot_dim & 1) ||
      rot_dim / 2 > kMaxRotHalf)
    return DSR_ERR_SHAPE;
  const int64_t row_bytes = (int64_t)head_dim * esize;
  if (row_bytes % 16 || page_bytes % row_bytes) return DSR_ERR_SHAPE;
  // Whole 16-byte vectors of rotated (and, neox, half-rotated) elements use
  // the vector kernels; other even rotary widths the LDS kernel.
  const bool vec_ok = ((int64_t)(head_dim - rot_dim) * esize) % 16 == 0 &&
                      (rope_style == DSR_ROPE_NEOX ? (rot_dim / 2) % ve == 0 : rot_dim % ve == 0);
  if (!vec_ok && row_bytes / 16 > 2048) return DSR_ERR_SHAPE;  // one row per LDS chunk
  // split-x K: a head's block of block_size tokens is the rotation "row";
  // only whole-vector rotary widths (the pair-task kernel) are supported
  if (kx_block < 0 || (kx_block > 0 && (!vec_ok || page_bytes % (row_bytes * kx_block))))
    return DSR_ERR_SHAPE;
  const int cd = kx_block > 0 ? kx_block : 1;
  const int task_vecs = !vec_ok ? 0 : rope_style == DSR_ROPE_NEOX ? rot_dim / 2 / ve
                                                                   : rot_dim / ve;
  if (n_pages == 0 || n_layers == 0) return DSR_OK;
  if (!rope_idx || (n_tables > 0 && !cos_sin)) return DSR_ERR_ARG;
  if (esize == 1 && !k_scale) return DSR_ERR_ARG;

  RotArgs ra{};
  ra.u = make_unit(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                   num_blocks, page_ids, slot_offsets, n_pages, staging,
                   staging_bytes, layer_bytes, layer0);
  ra.cos_sin = reinterpret_cast<const float2*>(cos_sin);
  ra.rope_idx = rope_idx;
  ra.n_tables = n_tables;
  ra.layer_group = layer_group;
  ra.n_groups = layer_group ? n_groups : 1;
  ra.row_vecs = (int)(row_bytes / 16) * cd;
  ra.rot_half = rot_dim / 2;
  ra.task_vecs = task_vecs * cd;
  ra.tail_vec0 = rot_dim * esize / 16 * cd;
  ra.tasks_per_row = (task_vecs + (head_dim - rot_dim) * esize / 16) * cd;
  ra.col_div = cd;
  ra.rot_vecs = rot_dim * esize / 16;
  ra.half_vecs = rope_style == DSR_ROPE_NEOX && vec_ok ? rot_dim / 2 * esize / 16 : 0;
  ra.k_scale = k_scale;
  hipStream_t s = (hipStream_t)stream;
  if (hnd_block > 0) {
    // head-major pages: the contig or grouped kernels (rows and partners
    // stay whole in record order; the cache side goes through hnd_vec)
    const int h = ra.half_vecs;
    const bool contig = vec_ok && (rope_style == DSR_ROPE_GPTJ ||
                                   (h > 0 && h <= 32 && (h & (h - 1)) == 0 &&
                                    ra.row_vecs % (2 * h) == 0));
    const int64_t rows = page_bytes / row_bytes;
    if (!contig || kx_block > 0 || rows % hnd_block) return DSR_ERR_SHAPE;
    ra.u.hnd_heads = (int)(rows / hnd_block);
    ra.u.hnd_block = hnd_block;
    ra.u.hnd_row_vecs = ra.row_vecs;
    switch (dtype) {
      case DSR_DTYPE_BF16:
        return launch_rerotate<DSR_DTYPE_BF16>(ra, n_pages, rope_style, true, s, false, flags,
                                               true);
      case DSR_DTYPE_FP16:
        return launch_rerotate<DSR_DTYPE_FP16>(ra, n_pages, rope_style, true, s, false, flags,
                                               true);
      case DSR_DTYPE_FP8_E4M3:
        return launch_rerotate<DSR_DTYPE_FP8_E4M3>(ra, n_pages, rope_style, true, s, false,
                                                   flags, true);
      default:
        return launch_rerotate<DSR_DTYPE_FP8_E5M2>(ra, n_pages, rope_style, true, s, false,
                                                   flags, true);
    }
  }
  if (kx_block > 0) {
    // vector kernels when the head block is a power-of-two number of
    // vectors (>= one wave), block_size a power of two and the neox partner
    // distance a multiple of 32 vectors (kx_phys); the pair-task kernel else
    const int64_t hv = row_bytes / 16 * kx_block;  // vectors per head block
    const int dist = rope_style == DSR_ROPE_NEOX ? task_vecs * kx_block : 0;
    const bool pow2 = (hv & (hv - 1)) == 0 && (kx_block & (kx_block - 1)) == 0;
    if (pow2 && hv >= kWave && dist % 32 == 0 && page_bytes % 1024 == 0 &&
        tune(DSR_TUNE_ROT_KERNEL) != kRotPairs) {
      ra.kx_row_shift = __builtin_ctzll((unsigned long long)hv);
      ra.kx_bs_shift = __builtin_ctz((unsigned)kx_block);
      ra.kx_dist = dist;
      ra.row_vecs = (int)hv;
      switch (dtype) {
        case DSR_DTYPE_BF16:
          return launch_rerotate<DSR_DTYPE_BF16>(ra, n_pages, rope_style, true, s, true, flags);
        case DSR_DTYPE_FP16:
          return launch_rerotate<DSR_DTYPE_FP16>(ra, n_pages, rope_style, true, s, true, flags);
        case DSR_DTYPE_FP8_E4M3:
          return launch_rerotate<DSR_DTYPE_FP8_E4M3>(ra, n_pages, rope_style, true, s, true, flags);
        default:
          return launch_rerotate<DSR_DTYPE_FP8_E5M2>(ra, n_pages, rope_style, true, s, true, flags);
      }
    }
    switch (dtype) {
      case DSR_DTYPE_BF16:
        return launch_rerotate_pairs<DSR_DTYPE_BF16>(ra, n_pages, rope_style, s);
      case DSR_DTYPE_FP16:
        return launch_rerotate_pairs<DSR_DTYPE_FP16>(ra, n_pages, rope_style, s);
      case DSR_DTYPE_FP8_E4M3:
        return launch_rerotate_pairs<DSR_DTYPE_FP8_E4M3>(ra, n_pages, rope_style, s);
      default:
        return launch_rerotate_pairs<DSR_DTYPE_FP8_E5M2>(ra, n_pages, rope_style, s);
    }
  }
  switch (dtype) {
    case DSR_DTYPE_BF16:
      return launch_rerotate<DSR_DTYPE_BF16>(ra, n_pages, rope_style, vec_ok, s, false, flags);
    case DSR_DTYPE_FP16:
      return launch_rerotate<DSR_DTYPE_FP16>(ra, n_pages, rope_style, vec_ok, s, false, flags);
    case DSR_DTYPE_FP8_E4M3:
      return launch_rerotate<DSR_DTYPE_FP8_E4M3>(ra, n_pages, rope_style, vec_ok, s, false, flags);
    default:
      return launch_rerotate<DSR_DTYPE_FP8_E5M2>(ra, n_pages, rope_style, vec_ok, s, false, flags);
  }
}

}  // namespace

extern "C" {

int dsr_scatter_rerotate(const uint64_t* layer_base, int n_layers,
                         int64_t kv_stride, int64_t page_stride,
                         int64_t page_bytes, int64_t num_blocks,
                         const int32_t* page_ids, const int64_t* slot_offsets,
                         int n_pages, const void* staging,
                         int64_t staging_bytes, int64_t layer_bytes,
                         int layer0, const float* cos_sin,
                         const int32_t* rope_idx, int n_tables,
                         const int32_t* layer_group, int n_groups, int head_dim,
                         int rot_dim, int rope_style, int dtype,
                         const float* k_scale, unsigned flags, dsr_stream_t stream) {
  return scatter_rerotate_any(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                              num_blocks, page_ids, slot_offsets, n_pages, staging,
                              staging_bytes, layer_bytes, layer0, cos_sin, rope_idx, n_tables,
                              layer_group, n_groups, head_dim, rot_dim, rope_style, dtype,
                              k_scale, 0, 0, flags, stream);
}

int dsr_scatter_rerotate_kx(const uint64_t* layer_base, int n_layers,
                            int64_t kv_stride, int64_t page_stride,
                            int64_t page_bytes, int64_t num_blocks,
                            const int32_t* page_ids, const int64_t* slot_offsets,
                            int n_pages, const void* staging,
                            int64_t staging_bytes, int64_t layer_bytes,
                            int layer0, const float* cos_sin,
                            const int32_t* rope_idx, int n_tables,
                            const int32_t* layer_group, int n_groups, int head_dim,
                            int rot_dim, int rope_style, int dtype,
                            const float* k_scale, int block_size, unsigned flags,
                            dsr_stream_t stream) {
  if (block_size <= 0) return DSR_ERR_ARG;
  return scatter_rerotate_any(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                              num_blocks, page_ids, slot_offsets, n_pages, staging,
                              staging_bytes, layer_bytes, layer0, cos_sin, rope_idx, n_tables,
                              layer_group, n_groups, head_dim, rot_dim, rope_style, dtype,
                              k_scale, block_size, 0, flags, stream);
}

int dsr_scatter_rerotate_hnd(const uint64_t* layer_base, int n_layers,
                             int64_t kv_stride, int64_t page_stride,
                             int64_t page_bytes, int64_t num_blocks,
                             const int32_t* page_ids, const int64_t* slot_offsets,
                             int n_pages, const void* staging,
                             int64_t staging_bytes, int64_t layer_bytes,
                             int layer0, const float* cos_sin,
                             const int32_t* rope_idx, int n_tables,
                             const int32_t* layer_group, int n_groups, int head_dim,
                             int rot_dim, int rope_style, int dtype,
                             const float* k_scale, int block_size, unsigned flags,
                             dsr_stream_t stream) {
  if (block_size <= 0) return DSR_ERR_ARG;
  return scatter_rerotate_any(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                              num_blocks, page_ids, slot_offsets, n_pages, staging,
                              staging_bytes, layer_bytes, layer0, cos_sin, rope_idx, n_tables,
                              layer_group, n_groups, head_dim, rot_dim, rope_style, dtype,
                              k_scale, 0, block_size, flags, stream);
}

}  // extern "C"

namespace {

// Head-major copies: the unit geometry, then one unit per workgroup.
int copy_hnd(bool gather, const uint64_t* layer_base, int n_layers, int64_t kv_stride,
             int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
             const int32_t* page_ids, const int64_t* slot_offsets, int n_pages,
             const void* staging, int64_t staging_bytes, int64_t layer_bytes, int layer0,
             int block_size, int num_heads, dsr_stream_t stream) {
  if (block_size <= 0 || num_heads <= 0) return DSR_ERR_ARG;
  int rc = check_common(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                        num_blocks, page_ids, slot_offsets, n_pages, staging,
                        staging_bytes, layer_bytes, layer0);
  if (rc != DSR_OK) return rc;
  const int64_t rows = (int64_t)block_size * num_heads;
  if (page_bytes % (rows * 16)) return DSR_ERR_SHAPE;
  if (n_pages == 0 || n_layers == 0) return DSR_OK;
  UnitArgs a = make_unit(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                         num_blocks, page_ids, slot_offsets, n_pages, staging,
                         staging_bytes, layer_bytes, layer0);
  a.hnd_heads = num_heads;
  a.hnd_block = block_size;
  a.hnd_row_vecs = (int)(page_bytes / rows / 16);
  // units per workgroup as for token-major pages (dsr_gather / dsr_scatter)
  const int G = gather ? (page_bytes < kThreads * 16
                              ? units_per_group(page_bytes, kGatherUnroll, kMaxGroup) : 1)
                       : (page_bytes <= kThreads * 16
                              ? units_per_group(page_bytes, kScatterUnroll, kMaxGroup) : 1);
  hipStream_t s = (hipStream_t)stream;
  return launch_page_ranges(a, n_pages, G, [&](const UnitArgs& b, unsigned grid) {
    if (G > 1 && gather)
      kv_copy_grouped_kernel<true, kGatherUnroll, true><<<grid, kThreads, 0, s>>>(b, G);
    else if (G > 1)
      kv_copy_grouped_kernel<false, kScatterUnroll, true><<<grid, kThreads, 0, s>>>(b, G);
    else if (gather)  // the page copies' occupancy policy: 11.26 vs 11.49 ms at
      kv_copy_hnd_kernel<true><<<grid, kThreads,  // config 2's pages head-major
                                 occupancy_lds(copy_wg_per_cu(page_bytes, b.n_units), 0), s>>>(b);
    else  // 12.52 vs 12.71 ms
      kv_copy_hnd_kernel<false><<<grid, kThreads,
                                  occupancy_lds(copy_wg_per_cu(page_bytes, b.n_units), 0), s>>>(b);
  });
}

}  // namespace

extern "C" {

int dsr_gather_hnd(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                   int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                   const int32_t* page_ids, const int64_t* slot_offsets, int n_pages,
                   void* staging, int64_t staging_bytes, int64_t layer_bytes, int layer0,
                   int block_size, int num_heads, dsr_stream_t stream) {
  return copy_hnd(true, layer_base, n_layers, kv_stride, page_stride, page_bytes, num_blocks,
                  page_ids, slot_offsets, n_pages, staging, staging_bytes, layer_bytes, layer0,
                  block_size, num_heads, stream);
}

int dsr_scatter_hnd(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                    int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                    const int32_t* page_ids, const int64_t* slot_offsets, int n_pages,
                    const void* staging, int64_t staging_bytes, int64_t layer_bytes,
                    int layer0, int block_size, int num_heads, dsr_stream_t stream) {
  return copy_hnd(false, layer_base, n_layers, kv_stride, page_stride, page_bytes,
                  num_blocks, page_ids, slot_offsets, n_pages, staging, staging_bytes,
                  layer_bytes, layer0, block_size, num_heads, stream);
}

}  // extern "C"

namespace {

// Unit order and workgroups per CU of the large-row token scatters
// (kv_slots_kernel, kv_slots_rerotate_kernel); DSR_TUNE_SLOTS_ORDER (1 per-XCD
// layer-major, 2 hardware dispatch order) and DSR_TUNE_SLOTS_WG_PER_CU
// override them.
bool slots_hw_order() { return tune(DSR_TUNE_SLOTS_ORDER) == 2; }
int slots_wg_per_cu(int dflt) {
  const int64_t t = tune(DSR_TUNE_SLOTS_WG_PER_CU);
  return t > 0 ? (int)t : dflt;
}

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
  if (const int64_t t = tune(DSR_TUNE_SLOTS_TPW))  // override for small rows
    if (tpw && (t == 4 || t == 8 || t == 16)) tpw = (int)t;
  // power-of-two rows of <= 8 vectors: the packed kernel, U instructions
  // per wave (4 and 8 measured alike; 16 spills)
  int pk_u = vpr <= 8 && (vpr & (vpr - 1)) == 0 && (block_size & (block_size - 1)) == 0 ? 8 : 0;
  if (tune(DSR_TUNE_SLOTS_KERNEL) == 1) pk_u = 0;
  if (const int64_t t = tune(DSR_TUNE_SLOTS_UNROLL))
    if (pk_u && (t == 4 || t == 8)) pk_u = (int)t;
  const int pk_s = pk_u ? __builtin_ctzll((unsigned long long)vpr) : 0;
  const int tok_wg = pk_u ? (kWave >> pk_s) * pk_u * (kThreads / kWave)
                     : tpw ? tpw * (kThreads / kWave) : kTokPerWg;
  const int64_t blocks = ((int64_t)n_tokens + tok_wg - 1) / tok_wg;
  if (blocks * n_layers > 0x7fffffffLL) return DSR_ERR_ARG;
  SlotArgs a{};
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
    if (pk_u == 8) {
      if (gather)
        kv_slots_packed_kernel<true, 8><<<grid, kThreads, 0, s>>>(b, pk_s);
      else
        kv_slots_packed_kernel<false, 8><<<grid, kThreads, 0, s>>>(b, pk_s);
    } else if (pk_u == 4) {
      if (gather)
        kv_slots_packed_kernel<true, 4><<<grid, kThreads, 0, s>>>(b, pk_s);
      else
        kv_slots_packed_kernel<false, 4><<<grid, kThreads, 0, s>>>(b, pk_s);
    } else if (tpw == 16) {
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
      kv_slots_kernel<true><<<grid, kThreads, occupancy_lds(3, 0), s>>>(b);
    } else if (slots_hw_order()) {
      kv_slots_kernel<false, true><<<grid, kThreads, occupancy_lds(slots_wg_per_cu(3), 0), s>>>(b);
    } else {
      kv_slots_kernel<false><<<grid, kThreads, occupancy_lds(slots_wg_per_cu(3), 0), s>>>(b);
    }
    const int rc = (int)hipGetLastError();
    if (rc != 0) return rc;
  }
  return DSR_OK;
}

// Token-form scatter with re-rotation: argument checks, then
// kv_slots_rerotate_kernel over token ranges that fit one launch each.
int slots_rerotate_launch(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                          int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                          int block_size, int64_t row_bytes, const int64_t* slot_mapping,
                          const int64_t* row_offsets, int n_tokens, const void* staging,
                          int64_t staging_bytes, int64_t layer_bytes, int layer0,
                          const float* cos_sin, const int32_t* rope_idx, int n_tables,
                          const int32_t* layer_group, int n_groups, int head_dim, int rot_dim,
                          int rope_style, int dtype, const float* k_scale, dsr_stream_t stream) {
  if (n_tokens < 0 || n_layers < 0 || layer0 < 0 || num_blocks < 0 || staging_bytes < 0 ||
      block_size <= 0 || row_bytes <= 0 || page_bytes <= 0 || n_tables < 0 ||
      (layer_group && n_groups < 1))
    return DSR_ERR_ARG;
  if (rope_style != DSR_ROPE_NEOX && rope_style != DSR_ROPE_GPTJ) return DSR_ERR_ARG;
  const int esize = dtype == DSR_DTYPE_BF16 || dtype == DSR_DTYPE_FP16 ? 2
                    : dtype == DSR_DTYPE_FP8_E4M3 || dtype == DSR_DTYPE_FP8_E5M2 ? 1 : 0;
  if (!esize) return DSR_ERR_ARG;
  if (n_tokens == 0 || n_layers == 0) return DSR_OK;
  if (!layer_base || !slot_mapping || !row_offsets || !staging || !rope_idx ||
      (n_tables > 0 && !cos_sin) || (esize == 1 && !k_scale))
    return DSR_ERR_ARG;
  // heads of a power-of-two number of vectors <= 64, rotary width in whole
  // vectors (both halves for neox), at most 256 rotated dims
  const int64_t head_bytes = (int64_t)head_dim * esize;
  const int ve = 16 / esize;
  const int hv = (int)(head_bytes / 16);
  if (head_dim <= 0 || rot_dim <= 0 || rot_dim > head_dim || rot_dim % 2 ||
      head_bytes % 16 || row_bytes % head_bytes || hv > kWave || (hv & (hv - 1)) ||
      rot_dim / 2 > kSlotRotMaxHalf ||
      (rope_style == DSR_ROPE_NEOX ? (rot_dim / 2) % ve : rot_dim % ve))
    return DSR_ERR_SHAPE;
  if (page_bytes < (int64_t)block_size * row_bytes || layer_bytes < 2 * page_bytes ||
      row_bytes > 0x7fffffffLL)
    return DSR_ERR_SHAPE;
  if (!aligned16(kv_stride) || !aligned16(page_stride) || !aligned16(page_bytes) ||
      !aligned16(row_bytes) || !aligned16(layer_bytes) || !aligned16p(staging))
    return DSR_ERR_ALIGN;
  const int64_t blocks = ((int64_t)n_tokens + kTokPerWg - 1) / kTokPerWg;
  if (blocks * n_layers > 0x7fffffffLL) return DSR_ERR_ARG;
  SlotArgs a{};
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
  RotArgs ra{};
  ra.u.layer0 = layer0;
  ra.cos_sin = reinterpret_cast<const float2*>(cos_sin);
  ra.rope_idx = rope_idx;
  ra.n_tables = n_tables;
  ra.layer_group = layer_group;
  ra.n_groups = layer_group ? n_groups : 1;
  ra.row_vecs = hv;
  ra.rot_half = rot_dim / 2;
  ra.rot_vecs = rot_dim * esize / 16;
  ra.half_vecs = rope_style == DSR_ROPE_NEOX ? rot_dim / 2 * esize / 16 : 0;
  ra.k_scale = k_scale;
  hipStream_t s = (hipStream_t)stream;
  const int64_t per = items_per_launch(n_layers, kTokPerWg) / kTokPerWg * kTokPerWg;
  if (per <= 0) return DSR_ERR_ARG;
  for (int64_t t0 = 0; t0 < n_tokens; t0 += per) {
    SlotArgs b = a;
    b.slot_mapping += t0;
    b.row_offsets += t0;
    b.n_tokens = (int32_t)(n_tokens - t0 < per ? n_tokens - t0 : per);
    RotArgs rb = ra;
    rb.rope_idx = rope_idx + t0;
    const int64_t units = ((int64_t)b.n_tokens + kTokPerWg - 1) / kTokPerWg * n_layers;
    const unsigned grid = (unsigned)((units + kXcds - 1) / kXcds * kXcds);
    const size_t dyn =
        occupancy_lds(slots_wg_per_cu(3), sizeof(float2) * kTokPerWg * kSlotRotMaxHalf);
    const bool neox = rope_style == DSR_ROPE_NEOX, hw = slots_hw_order();
#define DSR_SLOT_ROT(DT)                                                                      \
  (hw ? (neox ? kv_slots_rerotate_kernel<DT, DSR_ROPE_NEOX, true><<<grid, kThreads, dyn, s>>>(b, rb) \
              : kv_slots_rerotate_kernel<DT, DSR_ROPE_GPTJ, true><<<grid, kThreads, dyn, s>>>(b, rb)) \
      : (neox ? kv_slots_rerotate_kernel<DT, DSR_ROPE_NEOX><<<grid, kThreads, dyn, s>>>(b, rb)       \
              : kv_slots_rerotate_kernel<DT, DSR_ROPE_GPTJ><<<grid, kThreads, dyn, s>>>(b, rb)))
    switch (dtype) {
      case DSR_DTYPE_BF16: DSR_SLOT_ROT(DSR_DTYPE_BF16); break;
      case DSR_DTYPE_FP16: DSR_SLOT_ROT(DSR_DTYPE_FP16); break;
      case DSR_DTYPE_FP8_E4M3: DSR_SLOT_ROT(DSR_DTYPE_FP8_E4M3); break;
      default: DSR_SLOT_ROT(DSR_DTYPE_FP8_E5M2); break;
    }
#undef DSR_SLOT_ROT
    const int rc = (int)hipGetLastError();
    if (rc != 0) return rc;
  }
  return DSR_OK;
}

}  // namespace

extern "C" {

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

int dsr_scatter_slots_rerotate(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                               int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                               int block_size, int64_t row_bytes, const int64_t* slot_mapping,
                               const int64_t* row_offsets, int n_tokens, const void* staging,
                               int64_t staging_bytes, int64_t layer_bytes, int layer0,
                               const float* cos_sin, const int32_t* rope_idx, int n_tables,
                               const int32_t* layer_group, int n_groups, int head_dim,
                               int rot_dim, int rope_style, int dtype, const float* k_scale,
                               dsr_stream_t stream) {
  return slots_rerotate_launch(layer_base, n_layers, kv_stride, page_stride, page_bytes,
                               num_blocks, block_size, row_bytes, slot_mapping, row_offsets,
                               n_tokens, staging, staging_bytes, layer_bytes, layer0, cos_sin,
                               rope_idx, n_tables, layer_group, n_groups, head_dim, rot_dim,
                               rope_style, dtype, k_scale, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free load with re-rotation (dsr_scatter_rerotate_static).
//
// dsr_scatter_rerotate reads its tables (layer addresses, page ids, record
// offsets, table indices, angle tables, layer groups, scales) from device
// memory that the caller allocates per call. This variant takes them in host
// memory and stages them in `scratch`, a fixed device array of the library,
// then runs the same kernels on the staged copies. Each GPU holds its own
// copy of the array; its device address comes from hipGetSymbolAddress on
// the first call on that device (the array's name is a host-side stand-in
// and is never passed to a kernel or a copy).

namespace {

static __device__ __align__(256) uint8_t scratch[DSR_STATIC_TABLE_BYTES];

std::mutex g_scratch_mu;
uint8_t* g_scratch_ptr[kMaxDevices];  // per device, set once

// Device address of `scratch` on the current device (nullptr and *rc set
// on failure).
uint8_t* scratch_on_current_device(int* rc) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    *rc = (int)e;
    return nullptr;
  }
  if (dev < 0 || dev >= kMaxDevices) {
    *rc = DSR_ERR_ARG;
    return nullptr;
  }
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      *rc = e != hipSuccess ? (int)e : DSR_ERR_ARG;
      return nullptr;
    }
    g_scratch_ptr[dev] = static_cast<uint8_t*>(p);
  }
  return g_scratch_ptr[dev];
}

int64_t round256(int64_t v) { return (v + 255) & ~(int64_t)255; }

}  // namespace

extern "C" {

int dsr_scatter_rerotate_static(const uint64_t* layer_base, int n_layers,
                                int64_t kv_stride, int64_t page_stride,
                                int64_t page_bytes, int64_t num_blocks,
                                const int32_t* page_ids, const int64_t* slot_offsets,
                                int n_pages, const void* staging,
                                int64_t staging_bytes, int64_t layer_bytes,
                                int layer0, const float* cos_sin,
                                const int32_t* rope_idx, int n_tables,
                                const int32_t* layer_group, int n_groups, int head_dim,
                                int rot_dim, int rope_style, int dtype,
                                const float* k_scale, unsigned flags, dsr_stream_t stream) {
  if (n_pages < 0 || n_layers < 0 || layer0 < 0 || n_tables < 0 ||
      (layer_group && n_groups < 1))
    return DSR_ERR_ARG;
  if (n_pages == 0 || n_layers == 0) return DSR_OK;
  if (!layer_base || !page_ids || !slot_offsets || !rope_idx || (n_tables > 0 && !cos_sin))
    return DSR_ERR_ARG;
  if (rot_dim <= 0 || (rot_dim & 1) || rot_dim / 2 > kMaxRotHalf) return DSR_ERR_SHAPE;
  const int64_t rec_layers = (int64_t)layer0 + n_layers;  // entries of per-layer tables
  const int64_t groups = layer_group ? n_groups : 1;
  // packed sections of the staged tables, each 256-byte aligned
  const int64_t sz_base = (int64_t)n_layers * 8;
  const int64_t sz_ids = (int64_t)n_pages * 4;
  const int64_t sz_off = (int64_t)n_pages * 8;
  const int64_t sz_idx = (int64_t)n_pages * 4;
  const int64_t sz_cs = groups * n_tables * (rot_dim / 2) * 8;
  const int64_t sz_grp = layer_group ? rec_layers * 4 : 0;
  const int64_t sz_scl = k_scale ? rec_layers * 4 : 0;
  const int64_t o_base = 0, o_ids = o_base + round256(sz_base), o_off = o_ids + round256(sz_ids),
                o_idx = o_off + round256(sz_off), o_cs = o_idx + round256(sz_idx),
                o_grp = o_cs + round256(sz_cs), o_scl = o_grp + round256(sz_grp),
                total = o_scl + round256(sz_scl);
  if (total > DSR_STATIC_TABLE_BYTES) return DSR_ERR_TOO_LARGE;

  hipStream_t s = (hipStream_t)stream;
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t e = hipStreamIsCapturing(s, &cap);
  if (e != hipSuccess) return (int)e;
  if (cap != hipStreamCaptureStatusNone) return DSR_ERR_ARG;  // host-to-device copies

  int rc = DSR_OK;
  uint8_t* base = scratch_on_current_device(&rc);
  if (!base) return rc;
  struct Piece {
    int64_t off, bytes;
    const void* src;
  } pieces[] = {{o_base, sz_base, layer_base}, {o_ids, sz_ids, page_ids},
                {o_off, sz_off, slot_offsets}, {o_idx, sz_idx, rope_idx},
                {o_cs, sz_cs, cos_sin},       {o_grp, sz_grp, layer_group},
                {o_scl, sz_scl, k_scale}};
  for (const Piece& p : pieces) {
    if (p.bytes == 0) continue;
    e = hipMemcpyAsync(base + p.off, p.src, (size_t)p.bytes, hipMemcpyHostToDevice, s);
    if (e != hipSuccess) return (int)e;
  }
  return scatter_rerotate_any(
      reinterpret_cast<const uint64_t*>(base + o_base), n_layers, kv_stride, page_stride,
      page_bytes, num_blocks, reinterpret_cast<const int32_t*>(base + o_ids),
      reinterpret_cast<const int64_t*>(base + o_off), n_pages, staging, staging_bytes,
      layer_bytes, layer0, sz_cs ? reinterpret_cast<const float*>(base + o_cs) : nullptr,
      reinterpret_cast<const int32_t*>(base + o_idx), n_tables,
      layer_group ? reinterpret_cast<const int32_t*>(base + o_grp) : nullptr, n_groups,
      head_dim, rot_dim, rope_style, dtype,
      k_scale ? reinterpret_cast<const float*>(base + o_scl) : nullptr, 0, 0, flags, stream);
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Loads of shared records (dsr_scatter_fanout): one workgroup per (source
// record, layer), written to all of that record's destination pages.

namespace {

// Workgroups per CU of the fan-out kernel (DSR_TUNE_FANOUT_WG_PER_CU
// overrides): pages of 16 KiB and up at 2 (config 5's 32 KiB pages measured
// 33.58-33.64 ms from 2 to 8 per CU, 34.23 at 1), smaller ones at 8 (config
// 6's 4 KiB pages: 4.53 ms at 8, 4.55 at 4, 4.74 at 2, 6.54 at 1).
int fanout_wg_per_cu(int U) { return U >= 4 ? 2 : 8; }

template <int DT, int STYLE, int LAYOUT>
int launch_fanout_u(FanArgs fa, int U, int64_t n_src, hipStream_t s) {
  int wpc = fanout_wg_per_cu(U);
  if (const int64_t t = tune(DSR_TUNE_FANOUT_WG_PER_CU)) wpc = (int)t;
  const size_t dyn = occupancy_lds(
      wpc, (int64_t)sizeof(float2) * kFanLdsFloat2 + 2 * sizeof(int32_t) * kFanMaxBatch);
  // source ranges of at most max_wg_per_launch() workgroups each
  // (one source's layers and parts always fit HIP's limit; a tuning limit
  // below them still launches one source at a time)
  int64_t per = (max_wg_per_launch() - kXcds) / (fa.ra.u.n_layers * fa.parts);
  if (per <= 0) per = 1;
  for (int64_t s0 = 0; s0 < n_src; s0 += per) {
    FanArgs f = fa;
    const int64_t n = n_src - s0 < per ? n_src - s0 : per;
    f.src_offsets += s0;
    f.dst_start += s0;
    f.n_src = (int32_t)n;
    f.ra.u.n_units = n * fa.ra.u.n_layers;
    const unsigned grid = (unsigned)((f.ra.u.n_units * fa.parts + kXcds - 1) / kXcds * kXcds);
    switch (U) {
      case 1: kv_fanout_kernel<DT, STYLE, 1, LAYOUT><<<grid, kThreads, dyn, s>>>(f); break;
      case 2: kv_fanout_kernel<DT, STYLE, 2, LAYOUT><<<grid, kThreads, dyn, s>>>(f); break;
      case 4: kv_fanout_kernel<DT, STYLE, 4, LAYOUT><<<grid, kThreads, dyn, s>>>(f); break;
      default: kv_fanout_kernel<DT, STYLE, 8, LAYOUT><<<grid, kThreads, dyn, s>>>(f); break;
    }
    const int rc = (int)hipGetLastError();
    if (rc != 0) return rc;
  }
  return DSR_OK;
}

template <int DT, int LAYOUT>
int launch_fanout_l(const FanArgs& fa, int U, int64_t n_src, int style, hipStream_t s) {
  return style == DSR_ROPE_GPTJ ? launch_fanout_u<DT, DSR_ROPE_GPTJ, LAYOUT>(fa, U, n_src, s)
                                : launch_fanout_u<DT, DSR_ROPE_NEOX, LAYOUT>(fa, U, n_src, s);
}

template <int DT>
int launch_fanout(const FanArgs& fa, int U, int64_t n_src, int style, int layout,
                  hipStream_t s) {
  switch (layout) {
    case kFanKx: return launch_fanout_l<DT, kFanKx>(fa, U, n_src, style, s);
    case kFanHnd: return launch_fanout_l<DT, kFanHnd>(fa, U, n_src, style, s);
    default: return launch_fanout_l<DT, kFanNhd>(fa, U, n_src, style, s);
  }
}

}  // namespace

extern "C" {

int dsr_scatter_fanout(const uint64_t* layer_base, int n_layers, int64_t kv_stride,
                       int64_t page_stride, int64_t page_bytes, int64_t num_blocks,
                       const int64_t* src_offsets, int n_src, const int32_t* dst_start,
                       const int32_t* dst_page_ids, const int32_t* dst_rope_idx, int n_dst,
                       const void* staging, int64_t staging_bytes, int64_t layer_bytes,
                       int layer0, const float* cos_sin, int n_tables,
                       const int32_t* layer_group, int n_groups, int head_dim, int rot_dim,
                       int rope_style, int dtype, const float* k_scale, int k_layout,
                       int block_size, int num_heads, dsr_stream_t stream) {
  if (n_src < 0 || n_dst < 0) return DSR_ERR_ARG;
  if (k_layout != DSR_K_NHD && k_layout != DSR_K_KX && k_layout != DSR_K_HND) return DSR_ERR_ARG;
  if (k_layout != DSR_K_NHD && block_size <= 0) return DSR_ERR_ARG;
  // the page-table checks of the copies, with the destination ids and the
  // source offsets in the tables' places
  int rc = check_common(layer_base, n_layers, kv_stride, page_stride, page_bytes, num_blocks,
                        dst_page_ids, src_offsets, n_dst, staging, staging_bytes, layer_bytes,
                        layer0);
  if (rc != DSR_OK) return rc;
  // the geometry is checked before the empty-work return below, so that a
  // call with n_dst = 0 tells whether the fan-out takes a geometry
  // the page (or its part) in registers: at most 8 vectors per lane
  const int64_t nvec = page_bytes >> 4;
  if (nvec > 8 * kThreads) return DSR_ERR_SHAPE;
  RotArgs ra{};
  ra.u = make_unit(layer_base, n_layers, kv_stride, page_stride, page_bytes, num_blocks,
                   nullptr, nullptr, 0, staging, staging_bytes, layer_bytes, layer0);
  ra.n_groups = 1;
  ra.rot_half = 1;
  int dt = DSR_DTYPE_BF16, style = DSR_ROPE_NEOX;
  if (dst_rope_idx) {
    if (rope_style != DSR_ROPE_NEOX && rope_style != DSR_ROPE_GPTJ) return DSR_ERR_ARG;
    int esize, ve;
    switch (dtype) {
      case DSR_DTYPE_BF16:
      case DSR_DTYPE_FP16:
        esize = 2;
        ve = 8;
        break;
      case DSR_DTYPE_FP8_E4M3:
      case DSR_DTYPE_FP8_E5M2:
        esize = 1;
        ve = 16;
        break;
      default:
        return DSR_ERR_ARG;
    }
    if (n_tables < 0 || (layer_group && n_groups < 1)) return DSR_ERR_ARG;
    if (n_tables > 0 && !cos_sin) return DSR_ERR_ARG;
    if (esize == 1 && !k_scale) return DSR_ERR_ARG;
    if (head_dim <= 0 || rot_dim <= 0 || rot_dim > head_dim || (rot_dim & 1) ||
        rot_dim / 2 > kMaxRotHalf)
      return DSR_ERR_SHAPE;
    const int64_t row_bytes = (int64_t)head_dim * esize;
    if (row_bytes % 16 || page_bytes % row_bytes) return DSR_ERR_SHAPE;
    // the contig kernel's vector geometry: whole-vector rotary widths, neox
    // partners a power of two <= 32 vectors apart inside a row
    const bool vec_ok = ((int64_t)(head_dim - rot_dim) * esize) % 16 == 0 &&
                        (rope_style == DSR_ROPE_NEOX ? (rot_dim / 2) % ve == 0 : rot_dim % ve == 0);
    const int row_vecs = (int)(row_bytes / 16);
    const int h = rope_style == DSR_ROPE_NEOX && vec_ok ? rot_dim / 2 * esize / 16 : 0;
    const bool contig = vec_ok && (rope_style == DSR_ROPE_GPTJ ||
                                   (h > 0 && h <= 32 && (h & (h - 1)) == 0 &&
                                    row_vecs % (2 * h) == 0));
    if (!contig) return DSR_ERR_SHAPE;
    ra.cos_sin = reinterpret_cast<const float2*>(cos_sin);
    ra.n_tables = n_tables;
    ra.layer_group = layer_group;
    ra.n_groups = layer_group ? n_groups : 1;
    ra.row_vecs = row_vecs;
    ra.rot_half = rot_dim / 2;
    ra.rot_vecs = rot_dim * esize / 16;
    ra.half_vecs = h;
    ra.k_scale = k_scale;
    dt = dtype;
    style = rope_style;
    if (k_layout == DSR_K_KX) {
      // the contig kernel's split-x conditions: head blocks of a power-of-two
      // number (>= 64) of vectors, power-of-two block size, neox partners a
      // multiple of 32 vectors apart
      const int64_t hv = row_bytes / 16 * block_size;
      const int dist = rope_style == DSR_ROPE_NEOX ? rot_dim / 2 / ve * block_size : 0;
      if ((hv & (hv - 1)) || hv < kWave || (block_size & (block_size - 1)) || dist % 32 ||
          page_bytes % (row_bytes * block_size) || page_bytes % 1024)
        return DSR_ERR_SHAPE;
      ra.kx_row_shift = __builtin_ctzll((unsigned long long)hv);
      ra.kx_bs_shift = __builtin_ctz((unsigned)block_size);
      ra.kx_dist = dist;
      ra.row_vecs = (int)hv;
    } else if (k_layout == DSR_K_HND) {
      const int64_t rows = page_bytes / row_bytes;
      if (rows % block_size) return DSR_ERR_SHAPE;
      ra.u.hnd_heads = (int)(rows / block_size);
      ra.u.hnd_block = block_size;
      ra.u.hnd_row_vecs = row_vecs;
    }
  } else if (k_layout == DSR_K_HND) {
    // plain copy of head-major pages: rows of page_bytes / (block_size *
    // num_heads) bytes, whole vectors
    if (num_heads <= 0 || page_bytes % ((int64_t)block_size * num_heads * 16)) return DSR_ERR_SHAPE;
    ra.u.hnd_heads = num_heads;
    ra.u.hnd_block = block_size;
    ra.u.hnd_row_vecs = (int)(page_bytes / ((int64_t)block_size * num_heads) / 16);
  }
  // a plain copy of split-x pages moves raw bytes: the token-major kernel
  const int layout = k_layout == DSR_K_HND ? kFanHnd
                     : k_layout == DSR_K_KX && dst_rope_idx ? kFanKx : kFanNhd;
  // parts of whole rows (the rotation columns stay those of the page), at
  // least one vector per lane each
  int parts = 1;
  if (const int64_t t = tune(DSR_TUNE_FANOUT_PARTS)) parts = layout == kFanNhd ? (int)t : 1;
  const int64_t row_vecs = dst_rope_idx ? ra.row_vecs : 1;
  while (parts > 1 && (nvec % parts || (nvec / parts) % row_vecs || nvec / parts < kThreads))
    parts /= 2;
  if (parts < 1) parts = 1;
  if ((int64_t)n_src * n_layers * parts > 0x7fffffffLL) return DSR_ERR_ARG;
  const int64_t pv = nvec / parts;
  const int U = pv <= kThreads ? 1 : pv <= 2 * kThreads ? 2 : pv <= 4 * kThreads ? 4 : 8;
  if (n_src == 0 || n_dst == 0 || n_layers == 0) return DSR_OK;
  if (!dst_start) return DSR_ERR_ARG;
  FanArgs fa{};
  fa.ra = ra;
  fa.src_offsets = src_offsets;
  fa.dst_start = dst_start;
  fa.dst_pages = dst_page_ids;
  fa.dst_rope = dst_rope_idx;
  fa.n_src = n_src;
  fa.parts = parts;
  const int b = kFanLdsFloat2 / ra.rot_half;
  fa.batch = b < kFanMaxBatch ? b : kFanMaxBatch;
  hipStream_t s = (hipStream_t)stream;
  switch (dt) {
    case DSR_DTYPE_BF16: return launch_fanout<DSR_DTYPE_BF16>(fa, U, n_src, style, layout, s);
    case DSR_DTYPE_FP16: return launch_fanout<DSR_DTYPE_FP16>(fa, U, n_src, style, layout, s);
    case DSR_DTYPE_FP8_E4M3: return launch_fanout<DSR_DTYPE_FP8_E4M3>(fa, U, n_src, style, layout, s);
    default: return launch_fanout<DSR_DTYPE_FP8_E5M2>(fa, U, n_src, style, layout, s);
  }
}

}  // extern "C"
