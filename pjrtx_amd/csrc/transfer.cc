// Host-to-device uploads (and large device-to-host readbacks) through pinned
// staging (the reference's async H2D manager: src/plugin/async_h2d.zig,
// src/runtime/async_host_transfer.zig).
//
// A pageable host array is copied in chunks into a ring of pinned buffers
// by a few host threads while the DMA engine moves the previous chunk to
// the device on a copy stream of its own, so the host copy and the PCIe
// transfer overlap and each DMA reads pinned memory. The copy stream first
// waits for the device's compute stream: the destination block may have
// been freed by work still queued there (allocation is stream-ordered on
// that stream). The call returns when the data is on the device.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <map>
#include <memory>
#include <mutex>
#include <thread>
#include <vector>

#include "runtime.h"

namespace pjrtx {
namespace {

constexpr int kRing = 4;
constexpr size_t kChunk = 32u << 20;
constexpr int kCopyThreads = 4;

struct Stager {
  std::mutex mu;
  bool ready = false;
  hipStream_t stream = nullptr;
  hipEvent_t after_compute = nullptr;
  void* pinned[kRing] = {};
  hipEvent_t done[kRing] = {};
  bool busy[kRing] = {};
};

Stager& stager_for(int ordinal) {
  static std::mutex mu;
  static std::map<int, std::unique_ptr<Stager>> all;
  std::lock_guard<std::mutex> lk(mu);
  auto& s = all[ordinal];
  if (!s) s = std::make_unique<Stager>();
  return *s;
}

void init(Stager& st) {
  hip_check(hipStreamCreateWithFlags(&st.stream, hipStreamNonBlocking), "hipStreamCreate(copy)");
  hip_check(hipEventCreateWithFlags(&st.after_compute, hipEventDisableTiming), "hipEventCreate");
  for (int i = 0; i < kRing; ++i) {
    hip_check(hipHostMalloc(&st.pinned[i], kChunk, hipHostMallocDefault), "hipHostMalloc(staging)");
    hip_check(hipEventCreateWithFlags(&st.done[i], hipEventDisableTiming), "hipEventCreate");
  }
  st.ready = true;
}

// memcpy split over a few threads (one thread reaches ~10 GB/s from
// pageable memory; PCIe 5 x16 moves ~50).
void host_copy(void* dst, const void* src, size_t n) {
  if (n < (4u << 20)) {
    std::memcpy(dst, src, n);
    return;
  }
  // Parts rounded up (to whole pages): together they cover all n bytes.
  const size_t part = ((n + kCopyThreads - 1) / kCopyThreads + 4095) & ~size_t{4095};
  std::thread th[kCopyThreads - 1];
  for (int t = 1; t < kCopyThreads; ++t) {
    const size_t off = std::min(n, part * t), len = std::min(n - off, part);
    th[t - 1] = std::thread([=] { std::memcpy(static_cast<char*>(dst) + off, static_cast<const char*>(src) + off, len); });
  }
  std::memcpy(dst, src, std::min(n, part));
  for (auto& x : th) x.join();
}

}  // namespace

bool staged_upload_wanted(size_t bytes) {
  static const int on = env_int("PJRTX_STAGED_H2D", 1);
  // Measured crossover: HIP's own pageable copy is faster below ~64 MiB
  // (16 MiB: 31 vs 24 GB/s), the staged ring above (1 GiB: 54 vs 30 GB/s).
  return on != 0 && bytes >= (64u << 20);
}

void staged_upload(Device* dev, void* dst, const void* src, size_t bytes) {
  Stager& st = stager_for(dev->ordinal());
  std::lock_guard<std::mutex> lk(st.mu);
  dev->make_current();
  if (!st.ready) init(st);
  hip_check(hipEventRecord(st.after_compute, dev->stream()), "hipEventRecord");
  hip_check(hipStreamWaitEvent(st.stream, st.after_compute, 0), "hipStreamWaitEvent");
  int k = 0;
  for (size_t off = 0; off < bytes; off += kChunk, k = (k + 1) % kRing) {
    const size_t n = std::min(kChunk, bytes - off);
    if (st.busy[k]) hip_check(hipEventSynchronize(st.done[k]), "hipEventSynchronize(staging)");
    host_copy(st.pinned[k], static_cast<const char*>(src) + off, n);
    hip_check(hipMemcpyAsync(static_cast<char*>(dst) + off, st.pinned[k], n, hipMemcpyHostToDevice, st.stream),
              "hipMemcpyAsync(staged H2D)");
    hip_check(hipEventRecord(st.done[k], st.stream), "hipEventRecord");
    st.busy[k] = true;
  }
  hip_check(hipStreamSynchronize(st.stream), "hipStreamSynchronize(copy)");
  for (bool& b : st.busy) b = false;
}

bool staged_download_wanted(size_t bytes) {
  static const int on = env_int("PJRTX_STAGED_D2H", 1);
  return on != 0 && bytes >= (64u << 20);
}

// Device-to-host through the same ring: the DMA engine fills pinned chunk
// k+1.. while the host threads copy chunk k out to the caller's (pageable)
// memory. The copy stream first waits for the compute stream, which may
// still be producing the source.
void staged_download(Device* dev, void* dst, const void* src, size_t bytes) {
  Stager& st = stager_for(dev->ordinal());
  std::lock_guard<std::mutex> lk(st.mu);
  dev->make_current();
  if (!st.ready) init(st);
  hip_check(hipEventRecord(st.after_compute, dev->stream()), "hipEventRecord");
  hip_check(hipStreamWaitEvent(st.stream, st.after_compute, 0), "hipStreamWaitEvent");
  const size_t nchunks = (bytes + kChunk - 1) / kChunk;
  size_t issued = 0, copied = 0;
  while (copied < nchunks) {
    while (issued < nchunks && issued - copied < static_cast<size_t>(kRing)) {
      const size_t off = issued * kChunk, n = std::min(kChunk, bytes - off);
      const int k = static_cast<int>(issued % kRing);
      hip_check(hipMemcpyAsync(st.pinned[k], static_cast<const char*>(src) + off, n, hipMemcpyDeviceToHost, st.stream),
                "hipMemcpyAsync(staged D2H)");
      hip_check(hipEventRecord(st.done[k], st.stream), "hipEventRecord");
      ++issued;
    }
    const size_t off = copied * kChunk, n = std::min(kChunk, bytes - off);
    const int k = static_cast<int>(copied % kRing);
    hip_check(hipEventSynchronize(st.done[k]), "hipEventSynchronize(staging)");
    host_copy(static_cast<char*>(dst) + off, st.pinned[k], n);
    ++copied;
  }
  for (bool& b : st.busy) b = false;
}

// ------------------------------------------------------- async transfers

AsyncTransfer::AsyncTransfer(Device* dev, const std::vector<TensorType>& types) : dev_(dev) {
  for (const TensorType& t : types) {
    auto b = std::make_shared<Buffer>();
    b->dev = dev;
    b->type = t;
    b->mem = dev->allocate(t.bytes());
    auto ev = Event::pending();
    b->ready = ev;
    mems_.push_back(b->mem);
    bufs_.push_back(b);
    pending_.push_back(ev);
    finished_.push_back(false);
  }
}

size_t AsyncTransfer::bytes(size_t i) const {
  PJRTX_CHECK(i < bufs_.size(), Code::kInvalidArgument, "async transfer buffer index is out of range");
  return bufs_[i]->type.bytes();
}

BufferRef AsyncTransfer::buffer(size_t i) const {
  PJRTX_CHECK(i < bufs_.size(), Code::kInvalidArgument, "async transfer buffer index is out of range");
  return bufs_[i];
}

std::shared_ptr<Event> AsyncTransfer::write(size_t i, int64_t offset, const void* data, int64_t size, bool last) {
  std::lock_guard<std::mutex> lk(mu_);
  PJRTX_CHECK(i < bufs_.size(), Code::kInvalidArgument, "async transfer buffer index is out of range");
  PJRTX_CHECK(offset >= 0 && size >= 0, Code::kInvalidArgument, "async transfer offset and size must be non-negative");
  PJRTX_CHECK(data != nullptr || size == 0, Code::kInvalidArgument, "async transfer data is null");
  const size_t total = bufs_[i]->type.bytes();
  PJRTX_CHECK(static_cast<uint64_t>(offset) + static_cast<uint64_t>(size) <= total, Code::kInvalidArgument,
              "async transfer range exceeds buffer size");
  PJRTX_CHECK(!finished_[i], Code::kFailedPrecondition, "async transfer buffer already received its last chunk");
  PJRTX_CHECK(!bufs_[i]->deleted, Code::kFailedPrecondition, "async transfer buffer was deleted");
  dev_->make_current();
  std::shared_ptr<Event> done = Event::ready();
  if (size > 0) {
    char* dst = static_cast<char*>(mems_[i]->ptr) + offset;
    if (staged_upload_wanted(static_cast<size_t>(size))) {
      staged_upload(dev_, dst, data, static_cast<size_t>(size));  // returns once on the device
    } else {
      hip_check(hipMemcpyAsync(dst, data, static_cast<size_t>(size), hipMemcpyHostToDevice, dev_->stream()),
                "hipMemcpyAsync(async transfer)");
      done = Event::record(dev_);
    }
  }
  if (last) {
    finished_[i] = true;
    pending_[i]->resolve(Event::record(dev_));
    mems_[i].reset();  // the buffer alone owns its memory from here
  }
  return done;
}

AsyncTransfer::~AsyncTransfer() {
  std::lock_guard<std::mutex> lk(mu_);
  for (size_t i = 0; i < bufs_.size(); ++i)
    if (!finished_[i])
      pending_[i]->resolve_failed(Code::kCancelled, "async transfer manager destroyed before the buffer's last chunk");
}

void AsyncTransfer::fail(size_t i, Code code, const std::string& msg) {
  std::lock_guard<std::mutex> lk(mu_);
  PJRTX_CHECK(i < bufs_.size(), Code::kInvalidArgument, "async transfer buffer index is out of range");
  finished_[i] = true;
  pending_[i]->resolve_failed(code, msg);
  mems_[i].reset();
}

}  // namespace pjrtx
