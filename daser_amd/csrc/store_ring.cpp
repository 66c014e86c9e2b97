// store_ring.cpp -- pinned-host staging ring between device records and the
// DaseR store file, with an io_uring submission loop on the calling thread.
//
// Replaces the kvikio transfer layer of the reference
// (daser/connector/gds_transfer.py:22-127: CuFile.pwrite/pread of a GPU
// buffer, in compat mode a POSIX thread pool with a CPU bounce buffer).
//
// Write of n bytes at file offset F, in pieces of slot_bytes:
//   the side stream waits for the producer stream, then per piece k
//   (slot k % n_slots): hipMemcpyAsync device -> pinned slot, event e_k;
//   the caller waits e_k and submits an io_uring WRITE of the slot at
//   F + k * slot_bytes; a slot is refilled only after its write completed.
//   Copies of later pieces run on the GPU's DMA engine while earlier pieces
//   are being written.
// Read: the side stream waits for the consumer stream (earlier work may
//   still use the destination); io_uring READs fill free slots; each
//   completed read is copied pinned slot -> device on the side stream (event
//   e_k); a slot is reused after its copy event; the consumer stream waits
//   on the last copy.
//
// Without io_uring (ENOSYS/EPERM, or an op the kernel rejects) the same
// loop runs with pwrite/pread. Host mode (DSR_RING_HOST) uses plain memory
// and memcpy instead of pinned memory and HIP copies, which lets the I/O
// pipeline run without a GPU.
//
// Mapped mode (DSR_RING_MMAP): the file is mapped shared and a pool of
// worker threads copies between the pinned slots and the mapping. Buffered
// writes to one file serialise on the inode's lock in the kernel (one
// memcpy into the page cache at a time, about 17 GB/s on ext4 whatever the
// number of writer threads), while page faults on a shared mapping run in
// parallel; the device copies (PCIe, about 50 GB/s per direction) then set
// the pace. A write first allocates the blocks of its range (fallocate),
// so that a full file system fails with ENOSPC instead of faulting the
// process. Ranges past the end of the file go through the unmapped path.

#include <errno.h>
#include <fcntl.h>
#include <linux/falloc.h>
#include <linux/io_uring.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <sys/syscall.h>
#include <unistd.h>

#include <hip/hip_runtime_api.h>

#include <deque>
#include <thread>
#include <vector>

#include "daser_kv.h"

namespace {

// Minimal io_uring client over the kernel UAPI (no liburing): one submission
// at a time, completions reaped one by one.
class Uring {
 public:
  bool init(unsigned entries) {
    io_uring_params p;
    memset(&p, 0, sizeof(p));
    fd_ = (int)syscall(__NR_io_uring_setup, entries, &p);
    if (fd_ < 0) return false;
    sq_sz_ = p.sq_off.array + p.sq_entries * sizeof(unsigned);
    cq_sz_ = p.cq_off.cqes + p.cq_entries * sizeof(io_uring_cqe);
    sq_ptr_ = mmap(nullptr, sq_sz_, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd_,
                   IORING_OFF_SQ_RING);
    cq_ptr_ = mmap(nullptr, cq_sz_, PROT_READ | PROT_WRITE, MAP_SHARED | MAP_POPULATE, fd_,
                   IORING_OFF_CQ_RING);
    sqes_sz_ = p.sq_entries * sizeof(io_uring_sqe);
    sqes_ = (io_uring_sqe*)mmap(nullptr, sqes_sz_, PROT_READ | PROT_WRITE,
                                MAP_SHARED | MAP_POPULATE, fd_, IORING_OFF_SQES);
    if (sq_ptr_ == MAP_FAILED || cq_ptr_ == MAP_FAILED || sqes_ == MAP_FAILED) {
      close_all();
      return false;
    }
    char* sq = (char*)sq_ptr_;
    char* cq = (char*)cq_ptr_;
    sq_tail_ = (unsigned*)(sq + p.sq_off.tail);
    sq_mask_ = *(unsigned*)(sq + p.sq_off.ring_mask);
    sq_array_ = (unsigned*)(sq + p.sq_off.array);
    cq_head_ = (unsigned*)(cq + p.cq_off.head);
    cq_tail_ = (unsigned*)(cq + p.cq_off.tail);
    cq_mask_ = *(unsigned*)(cq + p.cq_off.ring_mask);
    cqes_ = (io_uring_cqe*)(cq + p.cq_off.cqes);
    return true;
  }

  // Queues and submits one READ/WRITE; returns 0 or -errno.
  int submit(int op, int file, void* buf, unsigned len, int64_t off, uint64_t tag) {
    const unsigned tail = *sq_tail_;
    const unsigned idx = tail & sq_mask_;
    io_uring_sqe* e = &sqes_[idx];
    memset(e, 0, sizeof(*e));
    e->opcode = (uint8_t)op;
    e->fd = file;
    e->addr = (uint64_t)(uintptr_t)buf;
    e->len = len;
    e->off = (uint64_t)off;
    e->user_data = tag;
    sq_array_[idx] = idx;
    __atomic_store_n(sq_tail_, tail + 1, __ATOMIC_RELEASE);
    for (;;) {
      const long r = syscall(__NR_io_uring_enter, fd_, 1, 0, 0, nullptr, 0);
      if (r >= 0) return 0;
      if (errno != EINTR) return -errno;
    }
  }

  // Waits for one completion; returns 0 or -errno of the wait itself.
  int wait(uint64_t* tag, int* res) {
    for (;;) {
      const unsigned head = *cq_head_;
      if (head != __atomic_load_n(cq_tail_, __ATOMIC_ACQUIRE)) {
        const io_uring_cqe& c = cqes_[head & cq_mask_];
        *tag = c.user_data;
        *res = c.res;
        __atomic_store_n(cq_head_, head + 1, __ATOMIC_RELEASE);
        return 0;
      }
      const long r = syscall(__NR_io_uring_enter, fd_, 0, 1, IORING_ENTER_GETEVENTS, nullptr, 0);
      if (r < 0 && errno != EINTR) return -errno;
    }
  }

  void close_all() {
    if (sqes_ && sqes_ != MAP_FAILED) munmap(sqes_, sqes_sz_);
    if (sq_ptr_ && sq_ptr_ != MAP_FAILED) munmap(sq_ptr_, sq_sz_);
    if (cq_ptr_ && cq_ptr_ != MAP_FAILED) munmap(cq_ptr_, cq_sz_);
    if (fd_ >= 0) ::close(fd_);
    fd_ = -1;
    sqes_ = nullptr;
    sq_ptr_ = cq_ptr_ = nullptr;
  }

 private:
  int fd_ = -1;
  void *sq_ptr_ = nullptr, *cq_ptr_ = nullptr;
  size_t sq_sz_ = 0, cq_sz_ = 0, sqes_sz_ = 0;
  io_uring_sqe* sqes_ = nullptr;
  io_uring_cqe* cqes_ = nullptr;
  unsigned *sq_tail_ = nullptr, *sq_array_ = nullptr, *cq_head_ = nullptr, *cq_tail_ = nullptr;
  unsigned sq_mask_ = 0, cq_mask_ = 0;
};

enum SlotState { kFree, kCopying, kIo, kLanded };

// One copy for the mapped mode's workers: wait `ev` (a slot's device copy),
// copy len bytes from src to dst, then mark `slot` (or nothing, -1) done.
struct CopyTask {
  int slot;
  hipEvent_t ev;
  uint8_t* dst;
  const uint8_t* src;
  int64_t len;
  bool write;
};

}  // namespace

struct dsr_ring {
  int fd = -1;
  int64_t slot_bytes = 0;
  int n_slots = 0;
  bool host = false;
  bool direct = false;  // O_DIRECT: offsets and lengths in kDirectAlign units
  bool use_uring = false;
  Uring uring;
  std::vector<uint8_t*> slots;
  std::vector<int> state;
  std::vector<hipEvent_t> ev;
  hipStream_t stream = nullptr;
  hipEvent_t ready = nullptr;
  pthread_mutex_t mu = PTHREAD_MUTEX_INITIALIZER;
  int last_errno = 0;
  // mapped mode
  bool mm = false;
  uint8_t* map = nullptr;
  int64_t map_len = 0;
  std::vector<std::thread> workers;
  pthread_mutex_t qmu = PTHREAD_MUTEX_INITIALIZER;
  pthread_cond_t qcv = PTHREAD_COND_INITIALIZER;  // a task was queued, or stop
  pthread_cond_t dcv = PTHREAD_COND_INITIALIZER;  // a task finished
  std::deque<CopyTask> queue;
  int64_t pending = 0;  // tasks queued or running
  int task_err = 0;     // first failure of a task (hipError_t, > 0)
  bool stop = false;
};

namespace {

// O_DIRECT transfers need file offsets, lengths and buffers aligned to the
// device's logical block; 4 KiB covers NVMe and the usual file systems.
constexpr int64_t kDirectAlign = 4096;
// Copy threads of the mapped mode (at most one per slot).
constexpr int kMaxCopyWorkers = 8;

bool direct_misaligned(const dsr_ring* r, int64_t nbytes, int64_t file_offset) {
  return r->direct && (nbytes % kDirectAlign || file_offset % kDirectAlign);
}

// Completes a transfer's piece synchronously (fallback path, or the rest of
// a short io_uring transfer). Returns 0 or -errno; 0 bytes read is -EIO.
int sync_io(dsr_ring* r, bool write, uint8_t* buf, int64_t len, int64_t off) {
  int64_t done = 0;
  while (done < len) {
    const ssize_t n = write ? pwrite(r->fd, buf + done, (size_t)(len - done), off + done)
                            : pread(r->fd, buf + done, (size_t)(len - done), off + done);
    if (n < 0) {
      if (errno == EINTR) continue;
      return -errno;
    }
    if (n == 0) return -EIO;
    done += n;
  }
  return 0;
}

// Starts the host I/O of one piece. With io_uring the piece completes later
// (reaped by reap_one); otherwise it completes here. Returns 0 or -errno.
int start_io(dsr_ring* r, bool write, int slot, int64_t len, int64_t off, int64_t piece,
             bool* async) {
  *async = false;
  if (r->use_uring) {
    const int rc = r->uring.submit(write ? IORING_OP_WRITE : IORING_OP_READ, r->fd,
                                   r->slots[slot], (unsigned)len, off,
                                   ((uint64_t)piece << 16) | (uint64_t)slot);
    if (rc == 0) {
      *async = true;
      return 0;
    }
    r->use_uring = false;  // submission refused: fall back for good
  }
  return sync_io(r, write, r->slots[slot], len, off);
}

struct Piece {
  int64_t len, off, dev_off;
};

// Reaps one io_uring completion: finishes a short transfer synchronously,
// falls back if the kernel rejects the op. Returns the completed slot and
// sets *err (0 or -errno).
int reap_one(dsr_ring* r, bool write, const std::vector<Piece>& pieces, int* err) {
  uint64_t tag = 0;
  int res = 0;
  *err = 0;
  const int w = r->uring.wait(&tag, &res);
  if (w < 0) {
    *err = w;
    return -1;
  }
  const int slot = (int)(tag & 0xffff);
  const Piece& pc = pieces[(size_t)(tag >> 16)];
  if (res == -EINVAL || res == -EOPNOTSUPP) {  // op unknown to this kernel
    r->use_uring = false;
    *err = sync_io(r, write, r->slots[slot], pc.len, pc.off);
  } else if (res < 0) {
    *err = res;
  } else if (res < pc.len) {
    if (!write && res == 0) {
      *err = -EIO;
    } else {
      *err = sync_io(r, write, r->slots[slot] + res, pc.len - res, pc.off + res);
    }
  }
  return slot;
}

int hip_rc(hipError_t e) { return e == hipSuccess ? 0 : (int)e; }

std::vector<Piece> split(int64_t n, int64_t slot_bytes, int64_t file_off) {
  std::vector<Piece> v;
  for (int64_t o = 0; o < n; o += slot_bytes)
    v.push_back({n - o < slot_bytes ? n - o : slot_bytes, file_off + o, o});
  return v;
}

// Makes slot s reusable: waits for its pending copy (reads) or I/O (writes).
int settle_slot(dsr_ring* r, int s, bool write, const std::vector<Piece>& pieces,
                int64_t* inflight) {
  int err = 0;
  while (r->state[s] == kIo) {  // reap until this slot's I/O is back
    int e = 0;
    const int done = reap_one(r, write, pieces, &e);
    if (done < 0) return e;
    if (e && !err) err = e;
    r->state[done] = kFree;
    --*inflight;
  }
  if (r->state[s] == kCopying) {
    if (!r->host) {
      const int e = hip_rc(hipEventSynchronize(r->ev[s]));
      if (e && !err) err = e;
    }
    r->state[s] = kFree;
  }
  return err;
}

// Mapped mode worker: runs copy tasks until the ring closes.
void worker_main(dsr_ring* r) {
  pthread_mutex_lock(&r->qmu);
  for (;;) {
    while (r->queue.empty() && !r->stop) pthread_cond_wait(&r->qcv, &r->qmu);
    if (r->queue.empty()) break;  // stop, and nothing left
    const CopyTask t = r->queue.front();
    r->queue.pop_front();
    pthread_mutex_unlock(&r->qmu);
    int e = 0;
    if (t.ev) e = hip_rc(hipEventSynchronize(t.ev));
    if (!e) memcpy(t.dst, t.src, (size_t)t.len);
    pthread_mutex_lock(&r->qmu);
    if (e && !r->task_err) r->task_err = e;
    if (t.slot >= 0) r->state[t.slot] = t.write ? kFree : kLanded;
    --r->pending;
    pthread_cond_broadcast(&r->dcv);
  }
  pthread_mutex_unlock(&r->qmu);
}

void enqueue(dsr_ring* r, const CopyTask& t) {
  pthread_mutex_lock(&r->qmu);
  if (t.slot >= 0) r->state[t.slot] = kIo;
  r->queue.push_back(t);
  ++r->pending;
  pthread_cond_signal(&r->qcv);
  pthread_mutex_unlock(&r->qmu);
}

// Waits (mapped mode) until slot s has no task queued or running; returns
// its state.
int wait_slot(dsr_ring* r, int s) {
  pthread_mutex_lock(&r->qmu);
  while (r->state[s] == kIo) pthread_cond_wait(&r->dcv, &r->qmu);
  const int st = r->state[s];
  pthread_mutex_unlock(&r->qmu);
  return st;
}

// Waits (mapped mode) for every queued task; returns and clears the first
// task failure.
int drain_tasks(dsr_ring* r) {
  pthread_mutex_lock(&r->qmu);
  while (r->pending > 0) pthread_cond_wait(&r->dcv, &r->qmu);
  const int e = r->task_err;
  r->task_err = 0;
  pthread_mutex_unlock(&r->qmu);
  return e;
}

// Maps the file so that [0, end) is covered. Returns 0 if mapped, 1 if the
// file is shorter than `end` (the caller takes the unmapped path), or
// -errno. Calls on a ring are serialised and no task runs between calls,
// so the old mapping can be replaced here.
int ensure_map(dsr_ring* r, int64_t end) {
  if (end <= r->map_len) return 0;
  struct stat st;
  if (fstat(r->fd, &st) != 0) return -errno;
  if ((int64_t)st.st_size < end) return 1;
  if (r->map) munmap(r->map, (size_t)r->map_len);
  r->map = nullptr;
  r->map_len = 0;
  void* m = mmap(nullptr, (size_t)st.st_size, PROT_READ | PROT_WRITE, MAP_SHARED, r->fd, 0);
  if (m == MAP_FAILED) return -errno;
  r->map = (uint8_t*)m;
  r->map_len = (int64_t)st.st_size;
  return 0;
}

// Before mapped writes to [off, off + n): its blocks are allocated (holes
// become unwritten extents, whose pages fault in as zeros without a disk
// read), so that a full file system is reported here (-ENOSPC) instead of
// as a fault on the mapping. A file system without fallocate is used as it
// is. (Deallocating the range first would spare the read of evicted pages
// on first touch, but ext4 writes a punched range's dirty pages back to
// the disk first: measured 2.5 GB/s saves against 15 with plain writes.)
int prepare_write_range(dsr_ring* r, int64_t off, int64_t n) {
  if (fallocate(r->fd, FALLOC_FL_KEEP_SIZE, off, n) != 0 && errno != EOPNOTSUPP &&
      errno != ENOSYS)
    return -errno;
  return 0;
}

// Mapped-mode write: device (or host) bytes -> pinned slots -> mapping,
// the copies into the mapping on the worker threads.
int mapped_write(dsr_ring* r, const void* src, const std::vector<Piece>& pieces,
                 hipStream_t producer) {
  const int64_t np = (int64_t)pieces.size(), S = r->n_slots;
  int err = 0;
  if (r->host) {  // host source: the workers copy straight into the mapping
    for (const Piece& pc : pieces)
      enqueue(r, {-1, nullptr, r->map + pc.off, (const uint8_t*)src + pc.dev_off, pc.len, true});
    return drain_tasks(r);
  }
  err = hip_rc(hipEventRecord(r->ready, producer));
  if (!err) err = hip_rc(hipStreamWaitEvent(r->stream, r->ready, 0));
  for (int64_t k = 0; k < np && !err; ++k) {
    const int s = (int)(k % S);
    wait_slot(r, s);  // its last piece is in the mapping
    const Piece& pc = pieces[(size_t)k];
    err = hip_rc(hipMemcpyAsync(r->slots[s], (const uint8_t*)src + pc.dev_off, (size_t)pc.len,
                                hipMemcpyDeviceToHost, r->stream));
    if (!err) err = hip_rc(hipEventRecord(r->ev[s], r->stream));
    if (!err) enqueue(r, {s, r->ev[s], r->map + pc.off, r->slots[s], pc.len, true});
  }
  const int e = drain_tasks(r);
  return err ? err : e;
}

// Mapped-mode read: mapping -> pinned slots (workers) -> device (the
// calling thread, in piece order, on the ring's stream).
int mapped_read(dsr_ring* r, void* dst, const std::vector<Piece>& pieces,
                hipStream_t consumer) {
  const int64_t np = (int64_t)pieces.size(), S = r->n_slots;
  int err = 0;
  if (r->host) {
    for (const Piece& pc : pieces)
      enqueue(r, {-1, nullptr, (uint8_t*)dst + pc.dev_off, r->map + pc.off, pc.len, false});
    return drain_tasks(r);
  }
  err = hip_rc(hipEventRecord(r->ready, consumer));
  if (!err) err = hip_rc(hipStreamWaitEvent(r->stream, r->ready, 0));
  int64_t queued = 0;
  for (int64_t k = 0; k < np && !err; ++k) {
    // keep every slot whose last device copy is done filling
    while (queued < np && queued - k < S && !err) {
      const int s = (int)(queued % S);
      if (r->state[s] == kCopying) {
        err = hip_rc(hipEventSynchronize(r->ev[s]));
        r->state[s] = kFree;
      }
      const Piece& pc = pieces[(size_t)queued];
      if (!err) enqueue(r, {s, nullptr, r->slots[s], r->map + pc.off, pc.len, false});
      ++queued;
    }
    if (err) break;
    const int s = (int)(k % S);
    if (wait_slot(r, s) != kLanded) break;  // a failed task: reported by the drain
    const Piece& pc = pieces[(size_t)k];
    err = hip_rc(hipMemcpyAsync((uint8_t*)dst + pc.dev_off, r->slots[s], (size_t)pc.len,
                                hipMemcpyHostToDevice, r->stream));
    if (!err) err = hip_rc(hipEventRecord(r->ev[s], r->stream));
    r->state[s] = kCopying;
  }
  const int e = drain_tasks(r);
  if (!err) err = e;
  if (!err) err = hip_rc(hipEventRecord(r->ready, r->stream));
  if (!err) err = hip_rc(hipStreamWaitEvent(consumer, r->ready, 0));
  return err;
}

}  // namespace

extern "C" {

int dsr_ring_open(const char* path, int64_t slot_bytes, int n_slots, int flags,
                  dsr_ring** out) {
  if (!path || !out || slot_bytes <= 0 || slot_bytes > 0x7fffffffLL || n_slots < 1 ||
      n_slots > 0xffff)
    return DSR_ERR_ARG;
  *out = nullptr;
  dsr_ring* r = new dsr_ring();
  r->slot_bytes = slot_bytes;
  r->n_slots = n_slots;
  r->host = (flags & DSR_RING_HOST) != 0;
  r->direct = (flags & DSR_RING_DIRECT) != 0;
  r->mm = (flags & DSR_RING_MMAP) != 0;
  if (r->direct && r->mm) {
    delete r;
    return DSR_ERR_ARG;
  }
  if (r->direct && slot_bytes % kDirectAlign) {
    delete r;
    return DSR_ERR_ALIGN;
  }
  r->fd = open(path, O_RDWR | O_CLOEXEC | ((flags & DSR_RING_DIRECT) ? O_DIRECT : 0));
  if (r->fd < 0) {
    r->last_errno = errno;
    const int e = errno == ENOENT ? DSR_ERR_NOFILE : DSR_ERR_IO;
    delete r;
    return e;
  }
  r->slots.assign((size_t)n_slots, nullptr);
  r->state.assign((size_t)n_slots, kFree);
  int rc = 0;
  for (int i = 0; i < n_slots && rc == 0; ++i) {
    // Pinned memory from hipHostMalloc is a driver mapping that O_DIRECT
    // cannot pin (the file operations fail with EFAULT), so direct mode
    // stages through aligned pageable slots and HIP's pageable copy path.
    if (r->host || r->direct) {
      if (posix_memalign((void**)&r->slots[i], 4096, (size_t)slot_bytes)) rc = DSR_ERR_ARG;
    } else {
      rc = hip_rc(hipHostMalloc((void**)&r->slots[i], (size_t)slot_bytes, hipHostMallocDefault));
    }
  }
  if (rc == 0 && !r->host) {
    rc = hip_rc(hipStreamCreateWithFlags(&r->stream, hipStreamNonBlocking));
    if (rc == 0) rc = hip_rc(hipEventCreateWithFlags(&r->ready, hipEventDisableTiming));
    r->ev.assign((size_t)n_slots, nullptr);
    for (int i = 0; i < n_slots && rc == 0; ++i)
      rc = hip_rc(hipEventCreateWithFlags(&r->ev[i], hipEventDisableTiming));
  }
  if (rc == 0 && !(flags & DSR_RING_NO_URING)) r->use_uring = r->uring.init((unsigned)n_slots * 2);
  if (rc == 0 && r->mm) {
    const int nw = n_slots < kMaxCopyWorkers ? n_slots : kMaxCopyWorkers;
    for (int i = 0; i < nw; ++i) r->workers.emplace_back(worker_main, r);
  }
  if (rc != 0) {
    dsr_ring_close(r);
    return rc;
  }
  *out = r;
  return DSR_OK;
}

int dsr_ring_uses_io_uring(const dsr_ring* r) { return r && r->use_uring ? 1 : 0; }

int dsr_ring_is_mapped(const dsr_ring* r) { return r && r->mm ? 1 : 0; }

int dsr_ring_last_errno(const dsr_ring* r) { return r ? r->last_errno : 0; }

int dsr_ring_write(dsr_ring* r, const void* src, int64_t nbytes, int64_t file_offset,
                   dsr_stream_t producer) {
  if (!r || (!src && nbytes) || nbytes < 0 || file_offset < 0) return DSR_ERR_ARG;
  if (nbytes == 0) return DSR_OK;
  if (direct_misaligned(r, nbytes, file_offset)) return DSR_ERR_ALIGN;
  pthread_mutex_lock(&r->mu);
  const std::vector<Piece> pieces = split(nbytes, r->slot_bytes, file_offset);
  if (r->mm) {
    int m = ensure_map(r, file_offset + nbytes);
    if (m == 0) m = prepare_write_range(r, file_offset, nbytes);
    if (m == 0) m = mapped_write(r, src, pieces, (hipStream_t)producer);
    if (m != 1) {  // 1: past the end of the file, written through pwrite below
      if (m < 0) {
        r->last_errno = -m;
        m = DSR_ERR_IO;
      }
      pthread_mutex_unlock(&r->mu);
      return m;
    }
  }
  const int64_t np = (int64_t)pieces.size(), S = r->n_slots;
  int err = 0;
  int64_t inflight = 0, copied = 0, submitted = 0;
  if (!r->host) {
    err = hip_rc(hipEventRecord(r->ready, (hipStream_t)producer));
    if (!err) err = hip_rc(hipStreamWaitEvent(r->stream, r->ready, 0));
  }
  while (!err && submitted < np) {
    // fill every slot that is free with the next pieces' copies
    while (!err && copied < np && copied - submitted < S) {
      const int s = (int)(copied % S);
      err = settle_slot(r, s, true, pieces, &inflight);
      if (err) break;
      const Piece& pc = pieces[(size_t)copied];
      const uint8_t* from = (const uint8_t*)src + pc.dev_off;
      if (r->host) {
        memcpy(r->slots[s], from, (size_t)pc.len);
      } else {
        err = hip_rc(hipMemcpyAsync(r->slots[s], from, (size_t)pc.len, hipMemcpyDeviceToHost,
                                    r->stream));
        if (!err) err = hip_rc(hipEventRecord(r->ev[s], r->stream));
      }
      r->state[s] = kCopying;
      ++copied;
    }
    if (err) break;
    // write the oldest copied piece
    const int s = (int)(submitted % S);
    if (!r->host) err = hip_rc(hipEventSynchronize(r->ev[s]));
    if (err) break;
    bool async = false;
    const Piece& pc = pieces[(size_t)submitted];
    err = start_io(r, true, s, pc.len, pc.off, submitted, &async);
    r->state[s] = async ? kIo : kFree;
    inflight += async ? 1 : 0;
    ++submitted;
  }
  // drain: every submitted write must be back before returning
  while (inflight > 0) {
    int e = 0;
    const int done = reap_one(r, true, pieces, &e);
    if (done < 0) {
      if (!err) err = e;
      break;
    }
    if (e && !err) err = e;
    r->state[done] = kFree;
    --inflight;
  }
  for (int s = 0; s < r->n_slots; ++s)
    if (r->state[s] == kCopying) {  // copies issued but never written (error path)
      if (!r->host) (void)hipEventSynchronize(r->ev[s]);  // already failing: best effort
      r->state[s] = kFree;
    }
  if (err < 0) {
    r->last_errno = -err;
    err = DSR_ERR_IO;
  }
  pthread_mutex_unlock(&r->mu);
  return err;
}

int dsr_ring_read(dsr_ring* r, void* dst, int64_t nbytes, int64_t file_offset,
                  dsr_stream_t consumer) {
  if (!r || (!dst && nbytes) || nbytes < 0 || file_offset < 0) return DSR_ERR_ARG;
  if (nbytes == 0) return DSR_OK;
  if (direct_misaligned(r, nbytes, file_offset)) return DSR_ERR_ALIGN;
  pthread_mutex_lock(&r->mu);
  const std::vector<Piece> pieces = split(nbytes, r->slot_bytes, file_offset);
  if (r->mm) {
    int m = ensure_map(r, file_offset + nbytes);
    if (m == 1) m = -EIO;  // past the end of the file
    if (m == 0) m = mapped_read(r, dst, pieces, (hipStream_t)consumer);
    if (m < 0) {
      r->last_errno = -m;
      m = DSR_ERR_IO;
    }
    pthread_mutex_unlock(&r->mu);
    return m;
  }
  const int64_t np = (int64_t)pieces.size(), S = r->n_slots;
  std::vector<int64_t> piece_of(S, -1);
  int err = 0;
  int64_t inflight = 0, submitted = 0, landed = 0;
  if (!r->host) {  // copies into dst wait for the consumer's earlier work on it
    err = hip_rc(hipEventRecord(r->ready, (hipStream_t)consumer));
    if (!err) err = hip_rc(hipStreamWaitEvent(r->stream, r->ready, 0));
  }
  auto land = [&](int s) -> int {  // a read is in slot s: copy it to the device
    const Piece& pc = pieces[(size_t)piece_of[s]];
    uint8_t* to = (uint8_t*)dst + pc.dev_off;
    ++landed;
    if (r->host) {
      memcpy(to, r->slots[s], (size_t)pc.len);
      r->state[s] = kFree;
      return 0;
    }
    int e = hip_rc(hipMemcpyAsync(to, r->slots[s], (size_t)pc.len, hipMemcpyHostToDevice,
                                  r->stream));
    if (!e) e = hip_rc(hipEventRecord(r->ev[s], r->stream));
    r->state[s] = kCopying;
    return e;
  };
  while (!err && landed < np) {
    // keep every free slot reading
    while (!err && submitted < np) {
      const int s = (int)(submitted % S);
      if (r->state[s] == kIo) break;  // its read has not landed yet
      err = settle_slot(r, s, false, pieces, &inflight);  // waits its last copy
      if (err) break;
      bool async = false;
      const Piece& pc = pieces[(size_t)submitted];
      piece_of[s] = submitted;
      err = start_io(r, false, s, pc.len, pc.off, submitted, &async);
      ++submitted;
      if (err) break;
      if (async) {
        r->state[s] = kIo;
        ++inflight;
      } else {
        err = land(s);
      }
    }
    if (err || inflight == 0) continue;
    int e = 0;
    const int s = reap_one(r, false, pieces, &e);
    if (s < 0) {
      err = e;
      break;
    }
    --inflight;
    if (e) {
      err = e;
      r->state[s] = kFree;
      break;
    }
    err = land(s);
  }
  while (inflight > 0) {  // error path: let in-flight reads finish
    int e = 0;
    const int s = reap_one(r, false, pieces, &e);
    if (s < 0) break;
    r->state[s] = kFree;
    --inflight;
  }
  if (!r->host) {
    int e = hip_rc(hipEventRecord(r->ready, r->stream));
    if (!e) e = hip_rc(hipStreamWaitEvent((hipStream_t)consumer, r->ready, 0));
    if (e && !err) err = e;
  }
  if (err < 0) {
    r->last_errno = -err;
    err = DSR_ERR_IO;
  }
  pthread_mutex_unlock(&r->mu);
  return err;
}

int dsr_ring_close(dsr_ring* r) {
  if (!r) return DSR_OK;
  int rc = 0;
  if (!r->workers.empty()) {
    pthread_mutex_lock(&r->qmu);
    r->stop = true;
    pthread_cond_broadcast(&r->qcv);
    pthread_mutex_unlock(&r->qmu);
    for (std::thread& t : r->workers) t.join();
  }
  if (r->map) munmap(r->map, (size_t)r->map_len);
  if (!r->host && r->stream) rc = hip_rc(hipStreamSynchronize(r->stream));
  r->uring.close_all();
  for (uint8_t* p : r->slots) {
    if (!p) continue;
    if (r->host || r->direct)
      free(p);
    else
      (void)hipHostFree(p);
  }
  for (hipEvent_t e : r->ev)
    if (e) (void)hipEventDestroy(e);
  if (r->ready) (void)hipEventDestroy(r->ready);
  if (r->stream) (void)hipStreamDestroy(r->stream);
  if (r->fd >= 0) ::close(r->fd);
  delete r;
  return rc;
}

}  // extern "C"
