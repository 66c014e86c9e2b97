// kv_slots.h -- token-granular (slot_mapping-driven) gather and scatter.
// Part of libdaser_kv: included by kv_move.hip, one translation unit.

#pragma once

#include "kv_common.h"
#include "kv_rotate.h"

namespace {

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

// Block of a non-negative slot: a shift for power-of-two block sizes (all
// of vLLM's), else a 32-bit division where the slot fits.
__device__ __forceinline__ int64_t slot_block(const SlotArgs& a, int64_t slot) {
  if (a.block_shift >= 0) return slot >> a.block_shift;
  return slot < (int64_t)0xffffffffLL ? udiv32(slot, a.block_size) : slot / a.block_size;
}

constexpr int kTokPerWave = 4;  // tokens whose rows a wave has in flight at once
constexpr int kTokPerWg = kTokPerWave * (kThreads / kWave);
constexpr int kRowUnroll = 2;   // 64-vector slices of a row per round

// One workgroup per (16 consecutive tokens, layer); each wave owns 4 of the
// tokens. Token addresses are wave-uniform (scalar loads of slot_mapping and
// row_offsets); the lanes cover a row's 16-byte vectors, so a wave moves a
// token's whole K and V rows, and 4 tokens' rows are in flight together.
// Branch-free over the rows: a padding or out-of-range token goes through
// zero-size descriptors (loads read 0, stores are dropped), and so do the
// vectors past a row, so each store is issued as soon as its own load has
// arrived (with a branch per vector the compiler waited for all 16 loads).
// Launched with dynamic LDS sized for three workgroups per CU, the
// registers' own limit: measured in-process at config 2, gather 12.04 ->
// 11.58 ms and scatter 12.63 -> 12.38 ms against the branching kernel
// without LDS (the branch-free kernel without LDS: 12.38 / 12.55; at one or
// two workgroups per CU: 13.8-14.3 ms).
template <bool kGather, bool kHwOrder = false>
__global__ __launch_bounds__(kThreads) void kv_slots_kernel(SlotArgs a) {
  // the scatter writes the paged cache: layer-major per XCD, as the page
  // scatter (-2.4% in-process), or layer-major in hardware dispatch order
  // (kHwOrder); the gather keeps the identity order
  int64_t unit = blockIdx.x;
  if (!kGather) {
    const int64_t nu = ((int64_t)a.n_tokens + kTokPerWg - 1) / kTokPerWg * a.n_layers;
    unit = kHwOrder ? layer_major_unit_hw(nu, a.n_layers) : layer_major_unit(nu, a.n_layers);
    if (unit < 0) return;
  }
  const int64_t tb = udiv32(unit, a.n_layers);
  const int l = (int)(unit - tb * a.n_layers);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int vpr = (int)(a.row_bytes >> 4);
  rsrc_t ck[kTokPerWave], cv[kTokPerWave], rk[kTokPerWave], rv[kTokPerWave];
#pragma unroll
  for (int j = 0; j < kTokPerWave; ++j) {
    const int64_t t = tb * kTokPerWg + wave * kTokPerWave + j;
    ck[j] = cv[j] = rk[j] = rv[j] = make_rsrc(a.staging, 0);
    if (t < a.n_tokens) {
      const int64_t slot = a.slot_mapping[t];
      const int64_t blk = slot >= 0 ? slot_block(a, slot) : -1;
      const int64_t off = a.row_offsets[t] + (int64_t)(a.layer0 + l) * a.layer_bytes;
      if (blk >= 0 && blk < a.num_blocks && off >= 0 &&
          off + a.page_bytes + a.row_bytes <= a.staging_bytes) {
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
        xk[j][m] = bload(kGather ? ck[j] : rk[j], v << 4);
        xv[j][m] = bload(kGather ? cv[j] : rv[j], v << 4);
      }
    }
#pragma unroll
    for (int j = 0; j < kTokPerWave; ++j) {
#pragma unroll
      for (int m = 0; m < kRowUnroll; ++m) {
        const int v = vb + m * kWave + lane;
        bstore(kGather ? rk[j] : ck[j], v << 4, xk[j][m]);
        bstore(kGather ? rv[j] : cv[j], v << 4, xv[j][m]);
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
  const int64_t tb = udiv32(unit, a.n_layers);
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
  const int64_t blk = slot < 0 ? -1 : slot_block(a, slot);
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

// Rows of 2^s <= 8 vectors (128 B: one e4m3 KV head of 128 dims, one bf16
// head of 64), packed 64 >> s tokens to a wave instruction: lane = (token
// sub-slot << s) | vector, so each load and store instruction moves a whole
// KiB (a token's row is contiguous on both sides), where the kernel above
// leaves 7/8 of its lanes idle on such rows. Measured on the e4m3 TP8 share
// (80 layers, 1 KV head, 2 KiB pages), two boxes: 5.2-5.3 / 5.1-5.9 TB/s
// gather / scatter against 3.6-3.8 / 3.5-3.7. At 16- and 32-vector rows it
// measured equal or slower than the kernel above (5.1-5.6 vs 5.3-5.7 TB/s
// gather), which keeps those. Each lane resolves
// its own token (the 2^s lanes of a token read the same table entries) and
// uses its own 64-bit global address; U instructions per wave are in flight
// for K and for V. Invalid tokens' lanes are masked off. Block sizes are
// powers of two here (vLLM's always are).
template <bool kGather, int U>
__global__ __launch_bounds__(kThreads, 4) void kv_slots_packed_kernel(SlotArgs a, int s) {
  const int tpi = kWave >> s;
  const int64_t tok_wg = (int64_t)tpi * U * (kThreads / kWave);
  int64_t unit = blockIdx.x;
  if (!kGather) {
    const int64_t nu = ((int64_t)a.n_tokens + tok_wg - 1) / tok_wg * a.n_layers;
    unit = layer_major_unit(nu, a.n_layers);
    if (unit < 0) return;
  }
  const int64_t tb = udiv32(unit, a.n_layers);
  const int l = (int)(unit - tb * a.n_layers);
  const int wave = (int)threadIdx.x / kWave, lane = (int)threadIdx.x % kWave;
  const int64_t vo = (int64_t)(lane & ((1 << s) - 1)) << 4;
  const int64_t t0 = tb * tok_wg + (int64_t)wave * tpi * U + (lane >> s);
  const uint8_t* base = reinterpret_cast<const uint8_t*>(a.layer_base[l]);
  const int64_t lofs = (int64_t)(a.layer0 + l) * a.layer_bytes;
  int64_t slot[U], roff[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {  // every table load first
    const int64_t t = t0 + (int64_t)k * tpi;
    const bool live = t < a.n_tokens;
    slot[k] = live ? a.slot_mapping[t] : -1;
    roff[k] = live ? a.row_offsets[t] : -1;
  }
  const int64_t sv = kGather ? a.kv_stride : a.page_bytes;  // K -> V, source side
  const int64_t dvs = kGather ? a.page_bytes : a.kv_stride;  // K -> V, destination side
  const uint8_t* src[U];
  uint8_t* dst[U];
  bool ok[U];
  u32x4 xk[U], xv[U];
#pragma unroll
  for (int k = 0; k < U; ++k) {
    // power-of-two block sizes only (the launcher checks): a shift and a mask
    const int64_t blk = slot[k] >> a.block_shift;  // -1 for padding slots
    const int64_t off = roff[k] + lofs;
    ok[k] = slot[k] >= 0 && blk < a.num_blocks && roff[k] >= 0 &&
            off + a.page_bytes + a.row_bytes <= a.staging_bytes;
    uint8_t* cache = const_cast<uint8_t*>(base) + blk * a.page_stride +
                     (slot[k] & (a.block_size - 1)) * a.row_bytes + vo;
    uint8_t* rec = a.staging + off + vo;
    src[k] = kGather ? cache : rec;
    dst[k] = kGather ? rec : cache;
    if (ok[k]) {
      xk[k] = *reinterpret_cast<const u32x4*>(src[k]);
      xv[k] = *reinterpret_cast<const u32x4*>(src[k] + sv);
    }
  }
#pragma unroll
  for (int k = 0; k < U; ++k) {
    if (ok[k]) {
      *reinterpret_cast<u32x4*>(dst[k]) = xk[k];
      *reinterpret_cast<u32x4*>(dst[k] + dvs) = xv[k];
    }
  }
}

// Token-form load scatter with the fused re-rotation: kv_slots_kernel's
// scatter (16 tokens per workgroup, 4 per wave, lanes across the row,
// branch-free) where the K vectors of a token with rope_idx[t] >= 0 go
// through rotate_vec with that token's (cos, sin) table. Each wave stages
// its own 4 tokens' tables in its slice of LDS with loads that write LDS
// directly (no registers), issued before the rows; one wait for all of the
// wave's loads then covers them. Heads are row_vecs (a power of two <= 64)
// vectors, so a head never straddles a 64-vector slice of the row and its
// neox partner sits half_vecs lanes away in the same load. At most 168
// VGPRs keep 3 waves per SIMD.
constexpr int kSlotRotMaxHalf = 128;  // rot_dim <= 256
// s_waitcnt vmcnt(0), expcnt and lgkmcnt left at their maxima
constexpr int kWaitVmcnt0 = 0x0F70;

template <int DT, int STYLE, bool kHwOrder = false>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3)))
void kv_slots_rerotate_kernel(SlotArgs a, RotArgs ra) {
  __shared__ float2 tab[kTokPerWg][kSlotRotMaxHalf];
  const int64_t nu = ((int64_t)a.n_tokens + kTokPerWg - 1) / kTokPerWg * a.n_layers;
  const int64_t unit =
      kHwOrder ? layer_major_unit_hw(nu, a.n_layers) : layer_major_unit(nu, a.n_layers);
  if (unit < 0) return;
  const int64_t tb = udiv32(unit, a.n_layers);
  const int l = (int)(unit - tb * a.n_layers);
  const int wave = threadIdx.x / kWave, lane = threadIdx.x % kWave;
  const int vpr = (int)(a.row_bytes >> 4);
  // layer l's group block of tables (-1: no RoPE in this layer)
  int gbase = 0;
  if (ra.layer_group) {
    const int g = ra.layer_group[ra.u.layer0 + l];
    gbase = g < 0 || g >= ra.n_groups ? -1 : g * ra.n_tables;
  }
  rsrc_t ck[kTokPerWave], cv[kTokPerWave], rk[kTokPerWave], rv[kTokPerWave];
  int ti[kTokPerWave];
#pragma unroll
  for (int j = 0; j < kTokPerWave; ++j) {
    const int64_t t = tb * kTokPerWg + wave * kTokPerWave + j;
    ck[j] = cv[j] = rk[j] = rv[j] = make_rsrc(a.staging, 0);
    ti[j] = -1;
    if (t < a.n_tokens) {
      const int64_t slot = a.slot_mapping[t];
      const int64_t ro = a.row_offsets[t];
      const int r = ra.rope_idx[t];
      const int64_t blk = slot >= 0 ? slot_block(a, slot) : -1;
      const int64_t off = ro + (int64_t)(a.layer0 + l) * a.layer_bytes;
      if (blk >= 0 && blk < a.num_blocks && off >= 0 &&
          off + a.page_bytes + a.row_bytes <= a.staging_bytes) {
        const uint8_t* row = reinterpret_cast<const uint8_t*>(a.layer_base[l]) +
                             blk * a.page_stride + (slot - blk * a.block_size) * a.row_bytes;
        ck[j] = make_rsrc(row, a.row_bytes);
        cv[j] = make_rsrc(row + a.kv_stride, a.row_bytes);
        rk[j] = make_rsrc(a.staging + off, a.row_bytes);
        rv[j] = make_rsrc(a.staging + off + a.page_bytes, a.row_bytes);
        ti[j] = r < 0 || r >= ra.n_tables || gbase < 0 ? -1 : gbase + r;
      }
    }
  }
  // this wave's tables straight into its LDS slice (16 bytes = 2 pairs per
  // lane: one load covers 128 pairs); zero-size descriptors for tokens that
  // keep their K
#pragma unroll
  for (int j = 0; j < kTokPerWave; ++j) {
    const uint8_t* tp = reinterpret_cast<const uint8_t*>(ra.cos_sin);
    const rsrc_t tr = ti[j] >= 0 ? make_rsrc(tp + (int64_t)ti[j] * ra.rot_half * sizeof(float2),
                                             ra.rot_half * (int64_t)sizeof(float2))
                                 : make_rsrc(tp, 0);
    __builtin_amdgcn_raw_ptr_buffer_load_lds(
        tr, (__attribute__((address_space(3))) void*)&tab[wave * kTokPerWave + j][0], 16,
        lane * 16, 0, 0, 0);
  }
  float scale = 1.0f, inv_scale = 1.0f;
  if (is_fp8<DT>()) {
    scale = ra.k_scale[a.layer0 + l];
    inv_scale = 1.0f / scale;
  }
  const int hv = ra.row_vecs;  // vectors per head
  // 64-vector slices per round: fp8 rows of up to 1 KiB fit one
  constexpr int RU = is_fp8<DT>() ? 1 : kRowUnroll;
  for (int vb = 0; vb < vpr; vb += kWave * RU) {
    u32x4 xk[kTokPerWave][RU], xv[kTokPerWave][RU];
#pragma unroll
    for (int j = 0; j < kTokPerWave; ++j) {
#pragma unroll
      for (int m = 0; m < RU; ++m) {
        const int v = vb + m * kWave + lane;
        xk[j][m] = bload(rk[j], v << 4);
        xv[j][m] = bload(rv[j], v << 4);
      }
    }
    if (vb == 0) {  // the tables (loaded first) and this round's rows have landed
      __builtin_amdgcn_s_waitcnt(kWaitVmcnt0);
      __builtin_amdgcn_wave_barrier();
      __atomic_signal_fence(__ATOMIC_SEQ_CST);  // no LDS read moves above the wait
    }
#pragma unroll
    for (int j = 0; j < kTokPerWave; ++j)
#pragma unroll
      for (int m = 0; m < RU; ++m) bstore(cv[j], (vb + m * kWave + lane) << 4, xv[j][m]);
#pragma unroll
    for (int j = 0; j < kTokPerWave; ++j) {
#pragma unroll
      for (int m = 0; m < RU; ++m) {
        const int v = vb + m * kWave + lane;
        u32x4 q = xk[j][m];
        if (STYLE == DSR_ROPE_NEOX) {  // the partner half_vecs away inside the same head
          const int c = v & (hv - 1);
          const int src = c < ra.half_vecs ? lane + ra.half_vecs : lane - ra.half_vecs;
#pragma unroll
          for (int x = 0; x < 4; ++x) q[x] = (unsigned)__shfl((int)xk[j][m][x], src);
        }
        const u32x4 r = rotate_vec<DT, STYLE>(ra, xk[j][m], q, v & (hv - 1),
                                              tab[wave * kTokPerWave + j], scale, inv_scale);
        bstore(ck[j], v << 4, ti[j] >= 0 ? r : xk[j][m]);
      }
    }
  }
}

}  // namespace
