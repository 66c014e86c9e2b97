// kv_fanout.h -- loads in which several pages read the same record (a cached
// chunk placed in several requests): each source record is read once and
// written to every page that loads it, K re-rotated per destination.
// Part of libdaser_kv: included by kv_move.hip, one translation unit.
//
// The per-page scatter reads a shared record once per destination page, so a
// chunk placed in 16 requests is read 16 times (partly from the memory-side
// cache). Here the unit is one (source record, layer): the workgroup loads
// the record's K and V pages into registers once, then for each destination
// stores V as is and K rotated by that destination's delta table. Reads drop
// to one pass over the distinct records; the writes are the same.

#pragma once

#include "kv_rotate.h"

namespace {

struct FanArgs {
  RotArgs ra;  // caches, staging, geometry, tables, scales (ra.u's page tables unused)
  const int64_t* src_offsets;  // n_src record offsets (layer 0 of the record)
  const int32_t* dst_start;    // n_src + 1: destinations of source s are [start[s], start[s+1])
  const int32_t* dst_pages;    // block id of each destination
  const int32_t* dst_rope;     // table index of each destination (-1: K copied); null: no rotation
  int32_t n_src;
  int32_t batch;  // destinations whose tables are staged in LDS at once
  int32_t parts;  // workgroups per unit, each a 1/parts share of whole rows of the page
};

constexpr int kFanLdsFloat2 = 2048;  // 16 KiB of staged (cos, sin) pairs
constexpr int kFanMaxBatch = 16;

// One workgroup per (source, layer), source-major (a source's layers are
// consecutive units) with each XCD taking one contiguous share of the units:
// an XCD reads its sources' records front to back, and the chip's writes at
// any moment spread over every layer's cache instead of one (config 5:
// 28.1 ms against 33.5 ms layer-major in hardware order, 28.5 ms source-major
// in hardware order). Pages of at most U * 4 KiB: the whole page sits in registers, U vectors per
// lane of K and of V. K rotation as in the contig kernel (neox partner from
// lane ^ half_vecs, fetched once per source since every destination rotates
// the same stored vectors).
// Cache layouts (LAYOUT): kFanNhd token-major pages; kFanKx split-x K pages
// of vLLM's 3-D PagedAttention caches (K vector i of the record is physical
// vector kx_phys(i) on both sides, neox partners lane ^ 32); kFanHnd
// head-major pages (records token-major: cache vector hnd_vec(i) for K and V,
// rotation columns in record order). kx and hnd units are whole pages.
constexpr int kFanNhd = 0, kFanKx = 1, kFanHnd = 2;

template <int DT, int STYLE, int U, int LAYOUT = kFanNhd>
__global__ __launch_bounds__(kThreads) void kv_fanout_kernel(FanArgs fa) {
  __shared__ float2 tabs[kFanLdsFloat2];
  __shared__ int32_t s_blk[kFanMaxBatch];
  __shared__ int32_t s_ti[kFanMaxBatch];
  const RotArgs& ra = fa.ra;
  const UnitArgs& a = ra.u;
  const int64_t w = xcd_unit(a.n_units * fa.parts);
  if (w < 0) return;
  // consecutive units take the parts of one (source, layer)
  const uint32_t b = (uint32_t)w / (uint32_t)fa.parts;
  const uint32_t part = (uint32_t)w - b * (uint32_t)fa.parts;
  const uint32_t s = b / (uint32_t)a.n_layers;
  const uint32_t l = b - s * (uint32_t)a.n_layers;
  const int64_t off = fa.src_offsets[s] + (int64_t)(a.layer0 + (int)l) * a.layer_bytes;
  const int d0 = fa.dst_start[s], d1 = fa.dst_start[s + 1];
  if (off < 0 || off + 2 * a.page_bytes > a.staging_bytes || d1 <= d0) return;
  const int64_t pb = a.page_bytes;
  // this part: whole rows, so a vector's rotation column is its index
  // modulo the row as in the whole page
  const int64_t sb = pb / fa.parts;
  const int64_t po = sb * part;
  const uint8_t* rec = a.staging + off + po;
  uint8_t* const lbase = reinterpret_cast<uint8_t*>(a.layer_base[l]) + po;
  const int nvec = (int)(sb >> 4);
  VRound<U> v, kk;
  v.load(make_rsrc(rec + pb, sb), threadIdx.x, nvec);
  if (LAYOUT == kFanKx)
    kk.load_kx(ra, make_rsrc(rec, sb), threadIdx.x, nvec);
  else
    kk.load(make_rsrc(rec, sb), threadIdx.x, nvec);
  // this layer's table block, or no rotation at all
  const int grp = ra.layer_group ? ra.layer_group[a.layer0 + (int)l] : 0;
  const bool rot_layer = fa.dst_rope != nullptr && grp >= 0 && grp < ra.n_groups;
  float scale = 1.0f, inv_scale = 1.0f;
  if (is_fp8<DT>() && rot_layer) {
    scale = ra.k_scale[a.layer0 + (int)l];
    inv_scale = 1.0f / scale;
  }
  u32x4 q[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    q[k] = kk.r[k];
    if (STYLE == DSR_ROPE_NEOX && rot_layer) {  // uniform: the whole wave shuffles
#pragma unroll
      for (int c = 0; c < 4; ++c)
        q[k][c] = (unsigned)__shfl_xor((int)kk.r[k][c], LAYOUT == kFanKx ? 32 : ra.half_vecs);
    }
  }
  const int rh = ra.rot_half;
  for (int db = d0; db < d1; db += fa.batch) {
    const int nb = d1 - db < fa.batch ? d1 - db : fa.batch;
    __syncthreads();  // the previous batch's tables and ids are no longer read
    if ((int)threadIdx.x < nb) {
      const int d = db + (int)threadIdx.x;
      s_blk[threadIdx.x] = fa.dst_pages[d];
      const int ti = rot_layer ? fa.dst_rope[d] : -1;
      s_ti[threadIdx.x] = ti >= 0 && ti < ra.n_tables ? grp * ra.n_tables + ti : -1;
    }
    __syncthreads();
    if (rot_layer) {
      for (int j = threadIdx.x; j < nb * rh; j += kThreads) {
        const int t = j / rh;
        const int ti = s_ti[t];
        tabs[j] = ti >= 0 ? ra.cos_sin[(int64_t)ti * rh + (j - t * rh)] : make_float2(1.0f, 0.0f);
      }
      __syncthreads();
    }
    for (int t = 0; t < nb; ++t) {
      const int64_t blk = s_blk[t];
      if (blk < 0 || blk >= a.num_blocks) continue;  // skipped, as by the page scatter
      uint8_t* const cache = lbase + blk * a.page_stride;
      const rsrc_t kd = make_rsrc(cache, sb), vd = make_rsrc(cache + a.kv_stride, sb);
      if (LAYOUT == kFanHnd)
        v.store_hnd(a, vd, threadIdx.x, nvec);
      else
        v.store(vd, threadIdx.x, nvec);
      const int ti = s_ti[t];
      const float2* tab = tabs + t * rh;
#pragma unroll
      for (int k = 0; k < U; ++k) {
        const int i = (int)threadIdx.x + k * kThreads;
        if (i >= nvec) continue;
        const int p = LAYOUT == kFanKx ? kx_phys(ra, i) : i;  // record-side vector
        const int o = LAYOUT == kFanHnd ? hnd_vec(a, i) : p;  // cache-side vector
        bstore(kd, o << 4,
               ti < 0 ? kk.r[k]
                      : rotate_vec<DT, STYLE>(ra, kk.r[k], q[k],
                                              k_column<LAYOUT == kFanKx>(ra, p), tab, scale,
                                              inv_scale));
      }
    }
  }
}

}  // namespace
