// C-ABI round trip without Python or torch: allocates a small paged cache with
// hipMalloc, gathers a permuted page list into slot records with dsr_gather,
// checks the records against a host memcpy of the same layout, scatters them
// into a second cache with dsr_scatter and checks the pages, then re-rotates
// with a zero table (rope_idx -1) through both K layouts' entry points and
// checks a bit-exact copy; gathers the page list from the cache read as
// head-major pages and checks the row permutation; gathers the
// same records token by token with dsr_gather_slots; writes them to a store
// file through the staging ring and reads them back. Exit code 0 on success;
// prints the failing check otherwise.
#include <fcntl.h>
#include <hip/hip_runtime_api.h>
#include <stdlib.h>
#include <unistd.h>

#include <cstdint>
#include <cstdio>
#include <cstring>
#include <vector>

#include "daser_kv.h"

#define REQUIRE(c, msg)                              \
  do {                                               \
    if (!(c)) {                                      \
      fprintf(stderr, "FAILED: %s (%s)\n", msg, #c); \
      return 1;                                      \
    }                                                \
  } while (0)

int main() {
  const int L = 3, NB = 9, bs = 16, H = 2, D = 64;
  const int64_t page = (int64_t)bs * H * D * 2, layer_bytes = 2 * page, slot = L * layer_bytes;
  const int64_t cache_bytes = 2 * NB * page;
  const int32_t ids[] = {7, 2, 5, 0};
  const int n = 4;
  std::vector<uint8_t> host(L * cache_bytes);
  for (size_t i = 0; i < host.size(); ++i) host[i] = (uint8_t)(i * 2654435761u >> 13);
  uint8_t *cache, *cache2, *stg;
  uint64_t* bases;
  int32_t* d_ids;
  int64_t* d_offs;
  REQUIRE(hipMalloc(&cache, L * cache_bytes) == hipSuccess, "hipMalloc");
  REQUIRE(hipMalloc(&cache2, L * cache_bytes) == hipSuccess, "hipMalloc");
  REQUIRE(hipMalloc(&stg, n * slot) == hipSuccess, "hipMalloc");
  REQUIRE(hipMalloc(&bases, 2 * L * sizeof(uint64_t)) == hipSuccess, "hipMalloc");
  REQUIRE(hipMalloc(&d_ids, sizeof(ids)) == hipSuccess, "hipMalloc");
  REQUIRE(hipMalloc(&d_offs, n * sizeof(int64_t)) == hipSuccess, "hipMalloc");
  std::vector<uint64_t> b(2 * L);
  std::vector<int64_t> offs(n);
  for (int l = 0; l < L; ++l) {
    b[l] = (uint64_t)(cache + l * cache_bytes);
    b[L + l] = (uint64_t)(cache2 + l * cache_bytes);
  }
  for (int p = 0; p < n; ++p) offs[p] = p * slot;
  hipMemcpy(cache, host.data(), host.size(), hipMemcpyHostToDevice);
  hipMemset(cache2, 0, L * cache_bytes);
  hipMemcpy(bases, b.data(), b.size() * 8, hipMemcpyHostToDevice);
  hipMemcpy(d_ids, ids, sizeof(ids), hipMemcpyHostToDevice);
  hipMemcpy(d_offs, offs.data(), n * 8, hipMemcpyHostToDevice);

  REQUIRE(dsr_abi_version() == DSR_ABI_VERSION, "abi version");
  int rc = dsr_gather(bases, L, NB * page, page, page, NB, d_ids, d_offs, n, stg, n * slot,
                      layer_bytes, 0, nullptr);
  REQUIRE(rc == 0, dsr_error_string(rc));
  std::vector<uint8_t> got(n * slot), want(n * slot);
  hipMemcpy(got.data(), stg, got.size(), hipMemcpyDeviceToHost);
  for (int p = 0; p < n; ++p)
    for (int l = 0; l < L; ++l) {
      const uint8_t* k = host.data() + l * cache_bytes + ids[p] * page;
      memcpy(want.data() + offs[p] + l * layer_bytes, k, page);
      memcpy(want.data() + offs[p] + l * layer_bytes + page, k + NB * page, page);
    }
  REQUIRE(got == want, "gather records");

  rc = dsr_scatter(bases + L, L, NB * page, page, page, NB, d_ids, d_offs, n, stg, n * slot,
                   layer_bytes, 0, nullptr);
  REQUIRE(rc == 0, dsr_error_string(rc));
  std::vector<uint8_t> c2(L * cache_bytes);
  hipMemcpy(c2.data(), cache2, c2.size(), hipMemcpyDeviceToHost);
  for (int l = 0; l < L; ++l)
    for (int blk = 0; blk < NB; ++blk)
      for (int kv = 0; kv < 2; ++kv) {
        const int64_t o = l * cache_bytes + kv * NB * page + blk * page;
        bool touched = false;
        for (int p = 0; p < n; ++p) touched |= ids[p] == blk;
        if (touched)
          REQUIRE(memcmp(c2.data() + o, host.data() + o, page) == 0, "scattered page");
        else
          for (int64_t i = 0; i < page; ++i) REQUIRE(c2[o + i] == 0, "untouched page");
      }

  // re-rotation entry point with every page unrotated: a bit-exact copy
  hipMemset(cache2, 0, L * cache_bytes);
  float* tab;
  int32_t* ridx;
  REQUIRE(hipMalloc(&tab, D / 2 * 2 * sizeof(float)) == hipSuccess, "hipMalloc");
  REQUIRE(hipMalloc(&ridx, n * sizeof(int32_t)) == hipSuccess, "hipMalloc");
  hipMemset(ridx, 0xff, n * sizeof(int32_t));
  rc = dsr_scatter_rerotate(bases + L, L, NB * page, page, page, NB, d_ids, d_offs, n, stg,
                            n * slot, layer_bytes, 0, tab, ridx, 1, nullptr, 0, D, D,
                            DSR_ROPE_NEOX,
                            DSR_DTYPE_BF16, nullptr, 0u, nullptr);
  REQUIRE(rc == 0, dsr_error_string(rc));
  std::vector<uint8_t> c3(L * cache_bytes);
  hipMemcpy(c3.data(), cache2, c3.size(), hipMemcpyDeviceToHost);
  REQUIRE(c3 == c2, "unrotated re-rotate scatter equals plain scatter");
  // the split-x entry point on the same bytes: unrotated pages are copied too
  hipMemset(cache2, 0, L * cache_bytes);
  rc = dsr_scatter_rerotate_kx(bases + L, L, NB * page, page, page, NB, d_ids, d_offs, n, stg,
                               n * slot, layer_bytes, 0, tab, ridx, 1, nullptr, 0, D, D,
                               DSR_ROPE_NEOX, DSR_DTYPE_BF16, nullptr, bs,
                               DSR_REROTATE_SHARED_RECORDS, nullptr);
  REQUIRE(rc == 0, dsr_error_string(rc));
  hipMemcpy(c3.data(), cache2, c3.size(), hipMemcpyDeviceToHost);
  REQUIRE(c3 == c2, "unrotated split-x re-rotate scatter equals plain scatter");
  REQUIRE(dsr_scatter_rerotate_kx(bases + L, L, NB * page, page, page, NB, d_ids, d_offs, n,
                                  stg, n * slot, layer_bytes, 0, tab, ridx, 1, nullptr, 0, D,
                                  D, DSR_ROPE_NEOX, DSR_DTYPE_BF16, nullptr, 0, 0u,
                                  nullptr) == DSR_ERR_ARG,
          "split-x without a block size rejected");

  REQUIRE(dsr_gather(bases, L, 4100, page, page, NB, d_ids, d_offs, n, stg, n * slot,
                     layer_bytes, 0, nullptr) == DSR_ERR_ALIGN,
          "misaligned stride rejected");

  // the same cache memory read as head-major pages ([H][bs][D]): records
  // hold each page's rows in token-major order, row (t, h) <- (h * bs + t)
  {
    const int64_t row = (int64_t)D * 2;
    uint8_t* stg3;
    REQUIRE(hipMalloc(&stg3, n * slot) == hipSuccess, "hipMalloc");
    rc = dsr_gather_hnd(bases, L, NB * page, page, page, NB, d_ids, d_offs, n, stg3, n * slot,
                        layer_bytes, 0, bs, H, nullptr);
    REQUIRE(rc == 0, dsr_error_string(rc));
    std::vector<uint8_t> got3(n * slot), want3(n * slot);
    hipMemcpy(got3.data(), stg3, got3.size(), hipMemcpyDeviceToHost);
    for (int p = 0; p < n; ++p)
      for (int l = 0; l < L; ++l)
        for (int kv = 0; kv < 2; ++kv) {
          const uint8_t* pg = host.data() + l * cache_bytes + kv * NB * page + ids[p] * page;
          uint8_t* rec = want3.data() + offs[p] + l * layer_bytes + kv * page;
          for (int t = 0; t < bs; ++t)
            for (int h = 0; h < H; ++h)
              memcpy(rec + (t * H + h) * row, pg + (h * bs + t) * row, row);
        }
    REQUIRE(got3 == want3, "head-major gather records");
    REQUIRE(dsr_gather_hnd(bases, L, NB * page, page, page, NB, d_ids, d_offs, n, stg3,
                           n * slot, layer_bytes, 0, 0, H, nullptr) == DSR_ERR_ARG,
            "head-major gather without a block size rejected");
    hipFree(stg3);
  }

  // token form: slot_mapping of the same pages, full pages -> the same records
  const int64_t row = (int64_t)H * D * 2;
  std::vector<int64_t> sm(n * bs), ro(n * bs);
  for (int p = 0; p < n; ++p)
    for (int t = 0; t < bs; ++t) {
      sm[p * bs + t] = (int64_t)ids[p] * bs + t;
      ro[p * bs + t] = offs[p] + t * row;
    }
  int64_t *d_sm, *d_ro;
  uint8_t* stg2;
  REQUIRE(hipMalloc(&d_sm, sm.size() * 8) == hipSuccess, "hipMalloc");
  REQUIRE(hipMalloc(&d_ro, ro.size() * 8) == hipSuccess, "hipMalloc");
  REQUIRE(hipMalloc(&stg2, n * slot) == hipSuccess, "hipMalloc");
  hipMemcpy(d_sm, sm.data(), sm.size() * 8, hipMemcpyHostToDevice);
  hipMemcpy(d_ro, ro.data(), ro.size() * 8, hipMemcpyHostToDevice);
  hipMemset(stg2, 0, n * slot);
  rc = dsr_gather_slots(bases, L, NB * page, page, page, NB, bs, row, d_sm, d_ro, n * bs, stg2,
                        n * slot, layer_bytes, 0, nullptr);
  REQUIRE(rc == 0, dsr_error_string(rc));
  std::vector<uint8_t> got2(n * slot);
  hipMemcpy(got2.data(), stg2, got2.size(), hipMemcpyDeviceToHost);
  REQUIRE(got2 == want, "slot_mapping gather equals page gather");

  // shared records, each read once (dsr_scatter_fanout): record p goes to
  // block ids[p] and records 0 and 2 also to blocks 1 and 3
  {
    const int64_t src_off[] = {0, slot, 2 * slot, 3 * slot};
    const int32_t start[] = {0, 2, 3, 5, 6};
    const int32_t dpages[] = {1, 7, 2, 3, 5, 0};
    int64_t* d_src;
    int32_t *d_start, *d_dp;
    REQUIRE(hipMalloc(&d_src, sizeof(src_off)) == hipSuccess, "hipMalloc");
    REQUIRE(hipMalloc(&d_start, sizeof(start)) == hipSuccess, "hipMalloc");
    REQUIRE(hipMalloc(&d_dp, sizeof(dpages)) == hipSuccess, "hipMalloc");
    hipMemcpy(d_src, src_off, sizeof(src_off), hipMemcpyHostToDevice);
    hipMemcpy(d_start, start, sizeof(start), hipMemcpyHostToDevice);
    hipMemcpy(d_dp, dpages, sizeof(dpages), hipMemcpyHostToDevice);
    hipMemset(cache2, 0, L * cache_bytes);
    rc = dsr_scatter_fanout(bases + L, L, NB * page, page, page, NB, d_src, 4, d_start, d_dp,
                            nullptr, 6, stg, n * slot, layer_bytes, 0, nullptr, 0, nullptr, 0,
                            0, 0, 0, 0, nullptr, DSR_K_NHD, 0, 0, nullptr);
    REQUIRE(rc == 0, dsr_error_string(rc));
    hipMemcpy(c3.data(), cache2, c3.size(), hipMemcpyDeviceToHost);
    std::vector<uint8_t> want3 = c2;  // the page scatter's result, plus blocks 1 and 3
    for (int l = 0; l < L; ++l)
      for (int kv = 0; kv < 2; ++kv) {
        const int64_t base = l * cache_bytes + kv * NB * page;
        memcpy(want3.data() + base + 1 * page, host.data() + base + ids[0] * page, page);
        memcpy(want3.data() + base + 3 * page, host.data() + base + ids[2] * page, page);
      }
    REQUIRE(c3 == want3, "fan-out load of shared records");
    // the geometry query: no work, null tables
    REQUIRE(dsr_scatter_fanout(bases + L, L, NB * page, page, 64 << 10, NB, nullptr, 0, nullptr,
                               nullptr, nullptr, 0, stg, 0, 128 << 10, 0, nullptr, 0, nullptr, 0,
                               0, 0, 0, 0, nullptr, DSR_K_NHD, 0, 0,
                               nullptr) == DSR_ERR_SHAPE,
            "fan-out refuses 64 KiB pages");
    hipFree(d_src);
    hipFree(d_start);
    hipFree(d_dp);
  }

  // the allocation-free load: host tables, staged in the library's own
  // device array; every page unrotated, so the plain scatter's bytes
  {
    std::vector<int32_t> h_ridx(n, -1);
    std::vector<float> h_tab(D, 0.0f);
    hipMemset(cache2, 0, L * cache_bytes);
    rc = dsr_scatter_rerotate_static(b.data() + L, L, NB * page, page, page, NB, ids,
                                     offs.data(), n, stg, n * slot, layer_bytes, 0, h_tab.data(),
                                     h_ridx.data(), 1, nullptr, 0, D, D, DSR_ROPE_NEOX,
                                     DSR_DTYPE_BF16, nullptr, 0u, nullptr);
    REQUIRE(rc == 0, dsr_error_string(rc));
    REQUIRE(hipDeviceSynchronize() == hipSuccess, "device sync");
    hipMemcpy(c3.data(), cache2, c3.size(), hipMemcpyDeviceToHost);
    REQUIRE(c3 == c2, "allocation-free load equals the plain scatter");
  }

  // staging ring: records -> store file at a slot offset -> back to the device
  char path[] = "/tmp/dsr_abi_XXXXXX";
  const int fd = mkstemp(path);
  REQUIRE(fd >= 0, "mkstemp");
  REQUIRE(ftruncate(fd, 8 * slot) == 0, "ftruncate");
  close(fd);
  dsr_ring* ring = nullptr;
  REQUIRE(dsr_ring_open("/tmp/dsr_abi_missing_file", page, 2, 0, &ring) == DSR_ERR_NOFILE,
          "missing store file rejected");
  rc = dsr_ring_open(path, page, 2, 0, &ring);  // pieces smaller than the transfer
  REQUIRE(rc == 0 && ring, dsr_error_string(rc));
  rc = dsr_ring_write(ring, stg, n * slot, 3 * slot, nullptr);
  REQUIRE(rc == 0, dsr_error_string(rc));
  hipMemset(stg2, 0, n * slot);
  rc = dsr_ring_read(ring, stg2, n * slot, 3 * slot, nullptr);
  REQUIRE(rc == 0, dsr_error_string(rc));
  REQUIRE(hipDeviceSynchronize() == hipSuccess, "device sync");
  hipMemcpy(got2.data(), stg2, got2.size(), hipMemcpyDeviceToHost);
  REQUIRE(got2 == want, "ring write/read round trip");
  REQUIRE(dsr_ring_read(ring, stg2, n * slot, 6 * slot, nullptr) == DSR_ERR_IO,
          "read past the end of the file");
  REQUIRE(dsr_ring_close(ring) == 0, "ring close");
  unlink(path);
  REQUIRE(hipDeviceSynchronize() == hipSuccess, "device sync");
  printf("abi_roundtrip ok\n");
  return 0;
}
