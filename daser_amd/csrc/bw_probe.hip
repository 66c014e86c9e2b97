// bw_probe.hip -- HBM ceiling probes for the measurements (libdaser_bwprobe.so).
//
// Not part of the KV path: bench.py --ceilings times these three plain
// streams on the same part, so that the page kernels' figures can be read
// against what the memory system sustains for each direction of traffic,
// not only against the 8 TB/s data-sheet peak:
//   read   every byte of a buffer once (16-byte buffer loads, nt policy),
//          folded into a per-lane xor that is stored only on an impossible
//          value (the loads cannot be dropped);
//   write  every byte of a buffer once (16-byte buffer stores, sc0 sc1, the
//          page kernels' store policy);
//   copy   src -> dst, both sequential, the page kernels' engine without the
//          page tables (all loads of a round, then its stores).
// One workgroup of 256 lanes per `unit` bytes; workgroups per CU are capped
// with dynamic LDS, as the page kernels' launch policy does.

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef unsigned int u32x4 __attribute__((ext_vector_type(4)));
typedef __amdgpu_buffer_rsrc_t rsrc_t;

constexpr int kThreads = 256;

__device__ __forceinline__ rsrc_t rsrc(const void* p, int64_t n) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), 0, (int)n, 0x00020000);
}

template <int U>
__global__ __launch_bounds__(kThreads) void probe_read(const uint8_t* src, int64_t unit,
                                                       uint32_t* sink) {
  const rsrc_t r = rsrc(src + (int64_t)blockIdx.x * unit, unit);
  u32x4 acc = {0, 0, 0, 0};
  for (int base = threadIdx.x; base < (int)(unit >> 4); base += kThreads * U) {
    u32x4 x[U];
#pragma unroll
    for (int k = 0; k < U; ++k) x[k] = __builtin_amdgcn_raw_buffer_load_b128(r, (base + k * kThreads) << 4, 0, 2);
#pragma unroll
    for (int k = 0; k < U; ++k) acc ^= x[k];
  }
  if ((acc.x ^ acc.y ^ acc.z ^ acc.w) == 0x9e3779b9u && acc.x == 0x7f4a7c15u)
    sink[threadIdx.x] = acc.y;
}

template <int U>
__global__ __launch_bounds__(kThreads) void probe_write(uint8_t* dst, int64_t unit) {
  const rsrc_t r = rsrc(dst + (int64_t)blockIdx.x * unit, unit);
  const u32x4 v = {threadIdx.x, blockIdx.x, 0x5a5a5a5au, 0};
  for (int base = threadIdx.x; base < (int)(unit >> 4); base += kThreads * U) {
#pragma unroll
    for (int k = 0; k < U; ++k)
      __builtin_amdgcn_raw_buffer_store_b128(v, r, (base + k * kThreads) << 4, 0, 17);
  }
}

// write-only to units at permuted places: workgroup g writes units
// g * per_wg ... + per_wg - 1 of the list, unit i at place perm[i]
template <int U>
__global__ __launch_bounds__(kThreads) void probe_write_perm(uint8_t* dst, int64_t unit,
                                                             const int32_t* perm, int per_wg) {
  const u32x4 v = {threadIdx.x, blockIdx.x, 0x5a5a5a5au, 0};
  for (int j = 0; j < per_wg; ++j) {
    const rsrc_t r = rsrc(dst + (int64_t)perm[(int64_t)blockIdx.x * per_wg + j] * unit, unit);
    for (int base = threadIdx.x; base < (int)(unit >> 4); base += kThreads * U) {
#pragma unroll
      for (int k = 0; k < U; ++k)
        __builtin_amdgcn_raw_buffer_store_b128(v, r, (base + k * kThreads) << 4, 0, 17);
    }
  }
}

template <int U>
__global__ __launch_bounds__(kThreads) void probe_copy(const uint8_t* src, uint8_t* dst,
                                                       int64_t unit) {
  const rsrc_t s = rsrc(src + (int64_t)blockIdx.x * unit, unit);
  const rsrc_t d = rsrc(dst + (int64_t)blockIdx.x * unit, unit);
  for (int base = threadIdx.x; base < (int)(unit >> 4); base += kThreads * U) {
    u32x4 x[U];
#pragma unroll
    for (int k = 0; k < U; ++k) x[k] = __builtin_amdgcn_raw_buffer_load_b128(s, (base + k * kThreads) << 4, 0, 2);
#pragma unroll
    for (int k = 0; k < U; ++k)
      __builtin_amdgcn_raw_buffer_store_b128(x[k], d, (base + k * kThreads) << 4, 0, 17);
  }
}

size_t lds_for(int wg_per_cu) {
  int dev = 0, lds = 0;
  if (wg_per_cu <= 0 || hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&lds, hipDeviceAttributeMaxSharedMemoryPerMultiprocessor, dev) !=
          hipSuccess)
    return 0;
  return (size_t)(lds / wg_per_cu / 512 * 512);
}

}  // namespace

extern "C" {

// op: 0 read, 1 write, 2 copy, 3 write with unit i at place src[i] (src: a
// permutation of the bytes / unit places, int32), one unit per workgroup;
// 4 the same with 16 units per workgroup. bytes a multiple of unit;
// unit a multiple of 4 KiB and at most 1 GiB; 16-byte aligned buffers.
// Returns 0, -1 for bad arguments, or a hipError_t.
int dsr_bw_probe(int op, const void* src, void* dst, int64_t bytes, int64_t unit,
                 int wg_per_cu, void* sink, hipStream_t stream) {
  if (op < 0 || op > 4 || unit < 4096 || unit % 4096 || unit > (1LL << 30) || bytes <= 0 ||
      bytes % unit || bytes / unit > 0x7fffffffLL)
    return -1;
  if ((op != 1 && !src) || (op != 0 && !dst) || (op == 0 && !sink)) return -1;
  if ((reinterpret_cast<uintptr_t>(src) | reinterpret_cast<uintptr_t>(dst)) & 15) return -1;
  const int per_wg = op == 4 ? 16 : 1;
  if ((bytes / unit) % per_wg) return -1;
  const unsigned grid = (unsigned)(bytes / unit / per_wg);
  const size_t lds = lds_for(wg_per_cu);
  // vectors per lane per round: the whole unit in one round up to 32 KiB
  const int64_t v = unit >> 12;
  const int U = v >= 8 && v % 8 == 0 ? 8 : v >= 4 && v % 4 == 0 ? 4 : v >= 2 && v % 2 == 0 ? 2 : 1;
  const uint8_t* s = static_cast<const uint8_t*>(src);
  uint8_t* d = static_cast<uint8_t*>(dst);
  uint32_t* k = static_cast<uint32_t*>(sink);
#define DSR_PROBE_LAUNCH(UU)                                                   \
  if (op == 0) probe_read<UU><<<grid, kThreads, lds, stream>>>(s, unit, k);    \
  else if (op == 1) probe_write<UU><<<grid, kThreads, lds, stream>>>(d, unit); \
  else if (op >= 3)                                                            \
    probe_write_perm<UU><<<grid, kThreads, lds, stream>>>(                     \
        d, unit, reinterpret_cast<const int32_t*>(s), per_wg);                 \
  else probe_copy<UU><<<grid, kThreads, lds, stream>>>(s, d, unit);
  switch (U) {
    case 8: DSR_PROBE_LAUNCH(8) break;
    case 4: DSR_PROBE_LAUNCH(4) break;
    case 2: DSR_PROBE_LAUNCH(2) break;
    default: DSR_PROBE_LAUNCH(1) break;
  }
#undef DSR_PROBE_LAUNCH
  const hipError_t e = hipGetLastError();
  return e == hipSuccess ? 0 : (int)e;
}

}  // extern "C"
