// Disk reader: positional reads of a GGUF file by a pool of worker threads,
// with reads destined for device memory copied out of pinned staging on the
// reader's copy stream as soon as they land.
//
// Replaces the reference's io/reader.py AsyncReader (a Python thread pool of
// seek + read, one file handle per thread) and the disk side of
// io/stream.py StreamingSource. Differences, all for the MI355X host path:
//   * O_DIRECT reads (4096-byte aligned spans into a page-aligned buffer of
//     the worker) where the file system allows it, so a streamed block skips
//     the page cache: one DMA from the drive, one memcpy into pinned
//     staging, one host-to-device copy;
//   * the host-to-device copy is queued by the worker that read the bytes,
//     so it overlaps the other workers' reads without a Python round trip;
//   * a read larger than one staging buffer is split into chunks that
//     different workers read in parallel (queue depth within one request).
// Pure host code: no kernels.
#include "nsx_common.h"

#include <errno.h>
#include <fcntl.h>
#include <stdlib.h>
#include <string.h>
#include <sys/stat.h>
#include <time.h>
#include <unistd.h>

#include <algorithm>
#include <atomic>
#include <condition_variable>
#include <deque>
#include <mutex>
#include <string>
#include <thread>
#include <unordered_map>
#include <vector>

namespace {

constexpr int64_t kAlign = 4096;  // O_DIRECT offset/length/buffer granule (a multiple of every logical block size)

double now_s() {
  timespec ts;
  clock_gettime(CLOCK_MONOTONIC, &ts);
  return (double)ts.tv_sec + 1e-9 * (double)ts.tv_nsec;
}

struct Slot {
  uint8_t* buf = nullptr;
  hipEvent_t copied = nullptr;  // recorded after the copy out of this buffer
  bool copy_pending = false;
};

struct Chunk {
  uint64_t ticket;
  int64_t off, len;  // file span
  uint8_t* dst;      // destination of the span's first byte
  bool device;
};

struct Ticket {
  int remaining = 0;
  bool device = false;
  bool failed = false;
  hipEvent_t done_ev = nullptr;  // recorded on the copy stream after the last chunk's copy
  std::string err;
};

}  // namespace

struct nsx_reader {
  std::string path;
  int fd_buffered = -1, fd_direct = -1;
  std::atomic<bool> direct{false};  // cleared by a worker if the file system refuses a direct read
  int64_t file_size = 0;
  int device = -1;
  hipStream_t copy_stream = nullptr;
  hipEvent_t order_ev = nullptr;  // orders the copy stream after the submitting stream
  int64_t slot_bytes = 0, chunk_bytes = 0;
  std::vector<Slot> slots;
  std::vector<int> free_slots;
  std::deque<Chunk> queue;
  std::unordered_map<uint64_t, Ticket> tickets;
  uint64_t next_ticket = 1;
  std::mutex mu;
  std::condition_variable cv_work, cv_done, cv_slot;
  std::vector<std::thread> workers;
  bool stop = false;
  nsx_reader_stats stats{};
};

namespace {

// Read file bytes [off, off + len) into `dst`. Direct reads go through the
// worker's `bounce` buffer (plain page-aligned memory: O_DIRECT cannot DMA
// into driver-pinned host memory, the kernel's page pinning refuses it), then
// one memcpy; buffered reads go straight to `dst` (the kernel copies out of
// its page cache), through `bounce` only if that copy faults. Returns the
// error text, empty on success.
std::string read_span(nsx_reader* r, int64_t off, int64_t len, uint8_t* dst, uint8_t* bounce) {
  if (r->direct.load()) {
    const int64_t a0 = off & ~(kAlign - 1), skew = off - a0;
    const int64_t want = skew + len, span = (want + kAlign - 1) & ~(kAlign - 1);
    int64_t got = 0;
    while (got < want) {
      const ssize_t n = pread(r->fd_direct, bounce + got, (size_t)(span - got), (off_t)(a0 + got));
      if (n < 0) {
        if (errno == EINTR) continue;
        if (errno == EINVAL && got == 0) {  // the file system refused this direct read: buffered from here on
          r->direct.store(false);
          return read_span(r, off, len, dst, bounce);
        }
        return std::string("read failed at ") + std::to_string(a0 + got) + ": " + strerror(errno);
      }
      if (n == 0) break;  // end of file
      got += n;
    }
    if (got < want)
      return "short read at " + std::to_string(off) + ": wanted " + std::to_string(len) + ", got " +
             std::to_string(got > skew ? got - skew : 0);
    memcpy(dst, bounce + skew, (size_t)len);
    return {};
  }
  uint8_t* out = dst;
  int64_t got = 0, base = 0;  // out[got - base] receives file byte off + got
  while (got < len) {
    const int64_t n_want = out == dst ? len - got : std::min(len - got, (int64_t)r->chunk_bytes);
    const ssize_t n = pread(r->fd_buffered, out + (got - base), (size_t)n_want, (off_t)(off + got));
    if (n < 0) {
      if (errno == EINTR) continue;
      if (errno == EFAULT && out == dst) {  // the destination refused the kernel's copy: bounce from here
        out = bounce;
        base = got;
        continue;
      }
      return std::string("read failed at ") + std::to_string(off + got) + ": " + strerror(errno);
    }
    if (n == 0) break;
    if (out != dst) {
      memcpy(dst + got, bounce, (size_t)n);
    }
    got += n;
    if (out != dst) base = got;
  }
  if (got < len)
    return "short read at " + std::to_string(off) + ": wanted " + std::to_string(len) + ", got " + std::to_string(got);
  return {};
}

void finish_chunk(nsx_reader* r, const Chunk& c, const std::string& err, double t0, double t1) {
  std::lock_guard<std::mutex> lk(r->mu);
  r->stats.read_seconds += t1 - t0;
  if (r->stats.first_read == 0.0 || t0 < r->stats.first_read) r->stats.first_read = t0;
  if (t1 > r->stats.last_read) r->stats.last_read = t1;
  auto it = r->tickets.find(c.ticket);
  if (it == r->tickets.end()) return;
  Ticket& t = it->second;
  if (!err.empty() && !t.failed) {
    t.failed = true;
    t.err = err;
  }
  if (err.empty()) r->stats.bytes_read += c.len;
  if (--t.remaining == 0) {
    // every chunk's copy of this ticket was queued on the copy stream before
    // its count came off (under this lock), so this event follows them all
    if (t.device && !t.failed && hipEventRecord(t.done_ev, r->copy_stream) != hipSuccess) {
      t.failed = true;
      t.err = "hipEventRecord on the copy stream failed";
    }
    r->cv_done.notify_all();
  }
}

void worker_main(nsx_reader* r) {
  if (r->device >= 0) (void)hipSetDevice(r->device);
  uint8_t* bounce = nullptr;  // this worker's direct-read buffer (slot_bytes, page aligned)
  if (posix_memalign((void**)&bounce, (size_t)kAlign, (size_t)r->slot_bytes) != 0) bounce = nullptr;
  while (true) {
    Chunk c;
    {
      std::unique_lock<std::mutex> lk(r->mu);
      r->cv_work.wait(lk, [&] { return r->stop || !r->queue.empty(); });
      if (r->stop) break;
      c = r->queue.front();
      r->queue.pop_front();
    }
    int si = -1;
    if (c.device) {  // device destinations go through a pinned staging slot
      std::unique_lock<std::mutex> lk(r->mu);
      r->cv_slot.wait(lk, [&] { return r->stop || !r->free_slots.empty(); });
      if (r->stop) break;
      si = r->free_slots.back();
      r->free_slots.pop_back();
    }
    Slot* slot = si >= 0 ? &r->slots[si] : nullptr;
    std::string err;
    if (!bounce) err = "no memory for the read buffer";
    if (slot && slot->copy_pending) {  // the previous copy out of this buffer must be done before it is overwritten
      if (hipEventSynchronize(slot->copied) != hipSuccess) err = "waiting for a staging copy failed";
      slot->copy_pending = false;
    }
    const double t0 = now_s();
    if (err.empty()) err = read_span(r, c.off, c.len, slot ? slot->buf : c.dst, bounce);
    const double t1 = now_s();
    if (err.empty() && c.device) {
      if (hipMemcpyAsync(c.dst, slot->buf, (size_t)c.len, hipMemcpyHostToDevice, r->copy_stream) != hipSuccess ||
          hipEventRecord(slot->copied, r->copy_stream) != hipSuccess)
        err = "queueing the host-to-device copy failed";
      else
        slot->copy_pending = true;
    }
    if (slot) {
      std::lock_guard<std::mutex> lk(r->mu);
      r->free_slots.push_back(si);
      r->cv_slot.notify_one();
    }
    finish_chunk(r, c, err, t0, t1);
  }
  free(bounce);
}

void destroy(nsx_reader* r) {
  {
    std::lock_guard<std::mutex> lk(r->mu);
    r->stop = true;
  }
  r->cv_work.notify_all();
  r->cv_slot.notify_all();
  for (auto& w : r->workers) w.join();
  for (auto& s : r->slots) {
    if (s.copied) {
      if (s.copy_pending) (void)hipEventSynchronize(s.copied);
      (void)hipEventDestroy(s.copied);
    }
    if (s.buf) (void)hipHostFree(s.buf);
  }
  for (auto& kv : r->tickets)
    if (kv.second.done_ev) (void)hipEventDestroy(kv.second.done_ev);
  if (r->order_ev) (void)hipEventDestroy(r->order_ev);
  if (r->fd_direct >= 0) close(r->fd_direct);
  if (r->fd_buffered >= 0) close(r->fd_buffered);
  if (r->device >= 0) (void)hipGetLastError();  // a host-only reader makes no HIP calls at all
  delete r;
}

}  // namespace

extern "C" int nsx_reader_open(const char* path, int n_workers, int flags, int n_slots, int64_t slot_bytes,
                               int device, void* copy_stream, nsx_reader** out) {
  NSX_REQUIRE(path && out, NSX_EINVAL, "null argument");
  NSX_REQUIRE(n_workers >= 0 && n_workers <= 256, NSX_EINVAL, "n_workers=%d outside 0..256", n_workers);
  NSX_REQUIRE(n_slots >= 1 && n_slots <= 4096, NSX_EINVAL, "n_slots=%d outside 1..4096", n_slots);
  NSX_REQUIRE(slot_bytes >= 3 * kAlign && slot_bytes % kAlign == 0 && slot_bytes <= (1ll << 30), NSX_EINVAL,
              "slot_bytes=%lld: a multiple of 4096 in [12288, 1 GiB]", (long long)slot_bytes);
  NSX_REQUIRE(device < 0 || copy_stream, NSX_EINVAL, "a device reader needs a copy stream");
  *out = nullptr;
  nsx_reader* r = new nsx_reader();
  r->path = path;
  r->device = device;
  r->copy_stream = (hipStream_t)copy_stream;
  r->slot_bytes = slot_bytes;
  r->chunk_bytes = slot_bytes - 2 * kAlign;  // room for the aligned span around any chunk
  r->fd_buffered = open(path, O_RDONLY | O_CLOEXEC);
  if (r->fd_buffered < 0) {
    const int e = errno;
    destroy(r);
    return nsx_fail(NSX_EIO, "cannot open %s: %s", path, strerror(e));
  }
  struct stat st;
  if (fstat(r->fd_buffered, &st) != 0 || !S_ISREG(st.st_mode)) {
    destroy(r);
    return nsx_fail(NSX_EIO, "%s is not a regular file", path);
  }
  r->file_size = (int64_t)st.st_size;
  if (flags & NSX_READ_DIRECT) {
    r->fd_direct = open(path, O_RDONLY | O_CLOEXEC | O_DIRECT);
    r->direct.store(r->fd_direct >= 0);  // tmpfs and some overlays refuse O_DIRECT: buffered reads then
  }
  r->slots.resize(device >= 0 ? (size_t)n_slots : 0);  // staging for device destinations only
  for (int i = 0; i < (int)r->slots.size(); ++i) {
    Slot& s = r->slots[(size_t)i];
    if (device >= 0) {
      if (hipHostMalloc((void**)&s.buf, (size_t)slot_bytes, hipHostMallocDefault) != hipSuccess ||
          hipEventCreateWithFlags(&s.copied, hipEventDisableTiming) != hipSuccess) {
        s.buf = nullptr;
        destroy(r);
        return nsx_fail(NSX_EHIP, "pinned staging allocation of %d x %lld bytes failed", n_slots,
                        (long long)slot_bytes);
      }
    }
    r->free_slots.push_back((int)r->slots.size() - 1 - i);
  }
  if (device >= 0 && hipEventCreateWithFlags(&r->order_ev, hipEventDisableTiming) != hipSuccess) {
    destroy(r);
    return nsx_fail(NSX_EHIP, "hipEventCreate failed");
  }
  r->stats.n_workers = n_workers;
  for (int i = 0; i < n_workers; ++i) r->workers.emplace_back(worker_main, r);
  *out = r;
  return NSX_OK;
}

extern "C" int nsx_reader_submit(nsx_reader* r, int64_t offset, int64_t nbytes, void* dst, int dst_on_device,
                                 void* stream, uint64_t* ticket) {
  NSX_REQUIRE(r && ticket, NSX_EINVAL, "null argument");
  NSX_REQUIRE(offset >= 0 && nbytes >= 0, NSX_EINVAL, "negative offset or size");
  NSX_REQUIRE(nbytes == 0 || dst, NSX_EINVAL, "null destination");
  NSX_REQUIRE(!dst_on_device || r->device >= 0, NSX_EINVAL, "this reader was opened for host destinations only");
  Ticket t;
  t.device = dst_on_device != 0;
  if (t.device) {
    NSX_HIP(hipEventCreateWithFlags(&t.done_ev, hipEventDisableTiming));
    // the copies must not overtake work already queued on the destination's stream
    std::lock_guard<std::mutex> lk(r->mu);
    if (hipEventRecord(r->order_ev, (hipStream_t)stream) != hipSuccess ||
        hipStreamWaitEvent(r->copy_stream, r->order_ev, 0) != hipSuccess) {
      (void)hipEventDestroy(t.done_ev);
      return nsx_fail(NSX_EHIP, "ordering the copy stream after the caller's stream failed");
    }
  }
  std::lock_guard<std::mutex> lk(r->mu);
  const uint64_t id = r->next_ticket++;
  const int64_t nchunk = nbytes == 0 ? 0 : nsx_cdiv(nbytes, r->chunk_bytes);
  t.remaining = (int)nchunk;
  if (nchunk == 0 && t.device && hipEventRecord(t.done_ev, r->copy_stream) != hipSuccess) {
    (void)hipEventDestroy(t.done_ev);
    return nsx_fail(NSX_EHIP, "hipEventRecord failed");
  }
  r->tickets.emplace(id, std::move(t));
  for (int64_t i = 0; i < nchunk; ++i) {
    const int64_t o = i * r->chunk_bytes;
    r->queue.push_back(Chunk{id, offset + o, std::min(r->chunk_bytes, nbytes - o), (uint8_t*)dst + o,
                             dst_on_device != 0});
  }
  r->stats.requests += 1;
  r->cv_work.notify_all();
  *ticket = id;
  return NSX_OK;
}

extern "C" int nsx_reader_poll(nsx_reader* r, uint64_t ticket) {
  if (!r) return -NSX_EINVAL;
  std::lock_guard<std::mutex> lk(r->mu);
  auto it = r->tickets.find(ticket);
  if (it == r->tickets.end()) return -NSX_EINVAL;
  return it->second.remaining == 0 ? 1 : 0;
}

extern "C" int nsx_reader_wait(nsx_reader* r, uint64_t ticket, int64_t timeout_us, void* stream) {
  NSX_REQUIRE(r, NSX_EINVAL, "null reader");
  std::unique_lock<std::mutex> lk(r->mu);
  auto it = r->tickets.find(ticket);
  NSX_REQUIRE(it != r->tickets.end(), NSX_EINVAL, "unknown or retired ticket %llu", (unsigned long long)ticket);
  auto ready = [&] { return it->second.remaining == 0; };
  if (timeout_us < 0) {
    r->cv_done.wait(lk, ready);
  } else if (!r->cv_done.wait_for(lk, std::chrono::microseconds(timeout_us), ready)) {
    return nsx_fail(NSX_ETIMEDOUT, "read of ticket %llu still pending after %lld us", (unsigned long long)ticket,
                    (long long)timeout_us);
  }
  Ticket t = std::move(it->second);
  r->tickets.erase(it);
  lk.unlock();
  int rc = NSX_OK;
  if (t.failed) {
    rc = nsx_fail(NSX_EIO, "%s: %s", r->path.c_str(), t.err.c_str());
  } else if (t.device && hipStreamWaitEvent((hipStream_t)stream, t.done_ev, 0) != hipSuccess) {
    rc = nsx_fail(NSX_EHIP, "hipStreamWaitEvent failed");
  }
  if (t.done_ev) {
    // destroying a recorded event is deferred by the runtime until it completes
    (void)hipEventDestroy(t.done_ev);
  }
  return rc;
}

extern "C" int nsx_reader_get_stats(nsx_reader* r, nsx_reader_stats* out) {
  NSX_REQUIRE(r && out, NSX_EINVAL, "null argument");
  std::lock_guard<std::mutex> lk(r->mu);
  *out = r->stats;
  out->direct = r->direct.load() ? 1 : 0;
  return NSX_OK;
}

extern "C" int nsx_reader_close(nsx_reader* r) {
  if (!r) return NSX_OK;
  {
    std::lock_guard<std::mutex> lk(r->mu);
    for (auto& c : r->queue) {  // dropped reads fail their tickets
      auto it = r->tickets.find(c.ticket);
      if (it != r->tickets.end()) {
        it->second.failed = true;
        it->second.err = "reader closed";
        --it->second.remaining;
      }
    }
    r->queue.clear();
  }
  destroy(r);
  return NSX_OK;
}
