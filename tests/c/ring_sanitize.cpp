// The staging ring (store_ring.cpp) in host mode, built with AddressSanitizer
// and UndefinedBehaviorSanitizer (host code only; no GPU): random transfer
// sizes and offsets through every slot geometry, io_uring, pread/pwrite and
// the mapped mode's worker threads,
// each read checked against what was written, and a read past the end of the
// file. Exit 0 and "ring sanitize ok" when clean; a sanitizer report aborts.
#include <fcntl.h>
#include <unistd.h>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>
#include <random>
#include "daser_kv.h"
int main() {
  char path[] = "/tmp/dsr_ring_san_XXXXXX";
  int fd = mkstemp(path); ftruncate(fd, 8 << 20); close(fd);
  std::mt19937 rng(1);
  for (int flags : {DSR_RING_HOST, DSR_RING_HOST | DSR_RING_NO_URING, DSR_RING_HOST | DSR_RING_MMAP}) {
    for (long slot : {4096L, 8192L, 65536L, 80000L}) {
      for (int ns : {1, 2, 3, 8}) {
        dsr_ring* r = nullptr;
        if (dsr_ring_open(path, slot, ns, flags, &r)) { printf("open fail\n"); return 1; }
        for (int it = 0; it < 30; ++it) {
          long n = 1 + rng() % 300000, off = rng() % ((8 << 20) - n);
          std::vector<unsigned char> a(n), b(n);
          for (auto& x : a) x = rng();
          if (dsr_ring_write(r, a.data(), n, off, nullptr)) { printf("write fail\n"); return 1; }
          if (dsr_ring_read(r, b.data(), n, off, nullptr)) { printf("read fail\n"); return 1; }
          if (memcmp(a.data(), b.data(), n)) { printf("mismatch\n"); return 1; }
        }
        std::vector<unsigned char> c(100);
        if (dsr_ring_read(r, c.data(), 100, (8 << 20) - 50, nullptr) != DSR_ERR_IO) { printf("eof\n"); return 1; }
        dsr_ring_close(r);
      }
    }
  }
  unlink(path);
  printf("ring sanitize ok\n");
  return 0;
}
