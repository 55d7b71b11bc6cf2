// Device runtime implementation. See runtime.h.
#include "runtime.h"
#include "kernels/library.h"
#include "kernels/noalloc.h"

#include <hip/hiprtc.h>
#include <sys/stat.h>
#include <unistd.h>

#include <chrono>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <fstream>
#include <set>
#include <sstream>

#include "fusion_device_inc.h"  // kFusionDeviceHeader (generated at build)

namespace pjrtx {

void hip_check(hipError_t e, const char* what) {
  if (e != hipSuccess) {
    fail(e == hipErrorOutOfMemory ? Code::kResourceExhausted : Code::kInternal,
         strformat("%s failed: %s", what, hipGetErrorString(e)));
  }
}

// ----------------------------------------------------------------- allocator

DeviceMemory::~DeviceMemory() {
  if (dev && ptr && !borrowed) dev->allocator().release(ptr, capacity);
}

namespace {
thread_local Arena* t_arena = nullptr;
}  // namespace

Arena* thread_arena() { return t_arena; }
ArenaScope::ArenaScope(Arena* a) : prev_(t_arena) { t_arena = a; }
ArenaScope::~ArenaScope() { t_arena = prev_; }

Allocator::~Allocator() = default;

static size_t round_capacity(size_t bytes) {
  if (bytes <= 4096) return 4096;
  if (bytes <= (size_t(1) << 20)) return (bytes + 4095) & ~size_t(4095);
  return (bytes + (size_t(1) << 20) - 1) & ~((size_t(1) << 20) - 1);
}

void* Allocator::alloc(size_t bytes, size_t* capacity) {
  const size_t cap = round_capacity(bytes);
  {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = free_.lower_bound(cap);
    if (it != free_.end() && it->first <= cap + cap / 4) {
      void* p = it->second;
      *capacity = it->first;
      free_.erase(it);
      in_use_ += static_cast<int64_t>(*capacity);
      if (in_use_ > peak_) peak_ = in_use_.load();
      num_allocs_++;
      if (static_cast<int64_t>(bytes) > largest_) largest_ = static_cast<int64_t>(bytes);
      return p;
    }
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, cap);
  if (e == hipErrorOutOfMemory) {
    (void)hipGetLastError();
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
    trim();
    e = hipMalloc(&p, cap);
  }
  hip_check(e, "hipMalloc");
  *capacity = cap;
  reserved_ += static_cast<int64_t>(cap);
  in_use_ += static_cast<int64_t>(cap);
  if (in_use_ > peak_) peak_ = in_use_.load();
  num_allocs_++;
  if (static_cast<int64_t>(bytes) > largest_) largest_ = static_cast<int64_t>(bytes);
  return p;
}

void Allocator::release(void* p, size_t capacity) {
  std::lock_guard<std::mutex> lk(mu_);
  free_.emplace(capacity, p);
  in_use_ -= static_cast<int64_t>(capacity);
}

void Allocator::trim() {
  std::lock_guard<std::mutex> lk(mu_);
  for (auto& [cap, p] : free_) {
    (void)hipFree(p);
    reserved_ -= static_cast<int64_t>(cap);
  }
  free_.clear();
}

// -------------------------------------------------------------------- device

Device::Device(int ordinal) : ordinal_(ordinal), alloc_(ordinal) {
  hip_check(hipSetDevice(ordinal), "hipSetDevice");
  hip_check(hipStreamCreateWithFlags(&stream_, hipStreamNonBlocking), "hipStreamCreate");
  hip_check(hipStreamCreateWithFlags(&aux_stream_, hipStreamNonBlocking), "hipStreamCreate(aux)");
  hip_check(hipEventCreateWithFlags(&fork_ev_, hipEventDisableTiming), "hipEventCreate(fork)");
  hip_check(hipEventCreateWithFlags(&join_ev_, hipEventDisableTiming), "hipEventCreate(join)");
  hip_check(hipStreamCreateWithFlags(&aux2_stream_, hipStreamNonBlocking), "hipStreamCreate(aux2)");
  hip_check(hipEventCreateWithFlags(&fork2_ev_, hipEventDisableTiming), "hipEventCreate(fork2)");
  hip_check(hipEventCreateWithFlags(&join2_ev_, hipEventDisableTiming), "hipEventCreate(join2)");
  hip_check(hipEventCreateWithFlags(&side_ev_, hipEventDisableTiming), "hipEventCreate(side)");
  xcd_round_robin_ = env_int("PJRTX_XCD_LOCAL", 1) != 0 && probe_xcd_round_robin(stream_);
  hip_check(hipMalloc(reinterpret_cast<void**>(&counters_), kArrivalCounterBytes), "hipMalloc(counters)");
  hip_check(hipMemsetAsync(counters_, 0, kArrivalCounterBytes, stream_), "hipMemsetAsync(counters)");
  hip_check(hipStreamSynchronize(stream_), "hipStreamSynchronize");
  hipDeviceProp_t prop;
  hip_check(hipGetDeviceProperties(&prop, ordinal), "hipGetDeviceProperties");
  arch_ = prop.gcnArchName;
  size_t colon = arch_.find(':');
  if (colon != std::string::npos) arch_ = arch_.substr(0, colon);
  name_ = prop.name;
  total_mem_ = static_cast<int64_t>(prop.totalGlobalMem);
  cus_ = prop.multiProcessorCount;
}

Device::~Device() {
  // Process-lifetime object; the stream is released with the process.
}

void Device::make_current() const { hip_check(hipSetDevice(ordinal_), "hipSetDevice"); }

hipEvent_t Device::take_event() {
  {
    std::lock_guard<std::mutex> lk(ev_mu_);
    if (!ev_free_.empty()) {
      hipEvent_t e = ev_free_.back();
      ev_free_.pop_back();
      return e;
    }
  }
  hipEvent_t e = nullptr;
  hip_check(hipEventCreateWithFlags(&e, hipEventDisableTiming), "hipEventCreate");
  return e;
}

void Device::give_event(hipEvent_t e) {
  std::lock_guard<std::mutex> lk(ev_mu_);
  ev_free_.push_back(e);
}

MemRef Device::allocate(size_t bytes) {
  auto m = std::make_shared<DeviceMemory>();
  m->dev = this;
  m->bytes = bytes;
  if (bytes == 0) return m;
  if (Arena* a = t_arena; a && a->dev == this) {
    const size_t off = (a->used + 255) & ~size_t(255);
    PJRTX_CHECK(off <= a->cap && bytes <= a->cap - off, Code::kResourceExhausted,
                strformat("allocation-free execute: the fixed device block of %zu bytes is too small (%zu bytes in "
                          "use, %zu more requested)",
                          a->cap, off, bytes));
    m->ptr = a->base + off;
    m->capacity = (bytes + 255) & ~size_t(255);
    m->borrowed = true;
    a->used = off + bytes;
    if (a->used > a->peak) a->peak = a->used;
    return m;
  }
  make_current();
  m->ptr = alloc_.alloc(bytes, &m->capacity);
  if (capture_pins_) capture_pins_->push_back(m);
  return m;
}

// --------------------------------------------------------------------- event

namespace {
// Runs on_ready callbacks once their events complete. Events on one stream
// complete in order, so a FIFO worker suffices.
class EventWorker {
 public:
  static EventWorker& get() {
    static EventWorker* w = new EventWorker();
    return *w;
  }
  void push(std::shared_ptr<Event> e, std::function<void()> fn) {
    std::lock_guard<std::mutex> lk(mu_);
    q_.emplace_back(std::move(e), std::move(fn));
    cv_.notify_one();
  }

 private:
  EventWorker() { std::thread([this] { loop(); }).detach(); }
  void loop() {
    while (true) {
      std::pair<std::shared_ptr<Event>, std::function<void()>> item;
      {
        std::unique_lock<std::mutex> lk(mu_);
        cv_.wait(lk, [&] { return !q_.empty(); });
        item = std::move(q_.front());
        q_.pop_front();
      }
      item.first->await();
      item.second();
    }
  }
  std::mutex mu_;
  std::condition_variable cv_;
  std::deque<std::pair<std::shared_ptr<Event>, std::function<void()>>> q_;
};
}  // namespace

std::shared_ptr<Event> Event::ready() {
  auto e = std::shared_ptr<Event>(new Event());
  e->done_ = true;
  return e;
}

std::shared_ptr<Event> Event::failed(Code code, const std::string& msg) {
  auto e = std::shared_ptr<Event>(new Event());
  e->done_ = true;
  e->code_ = code;
  e->msg_ = msg;
  return e;
}

// The event is lazy: a hipEventRecord after every execution costs the host
// more than a kernel launch and stops HIP from batching the launches that
// follow, and most results are never asked whether they are ready. The
// hipEvent is recorded when readiness is first asked for; it then marks a
// stream position at or after this work, and the stream runs in order, so
// readiness is never reported before the work is done (at worst after some
// later work too).
std::shared_ptr<Event> Event::record(Device* dev) {
  auto e = std::shared_ptr<Event>(new Event());
  e->dev_ = dev;
  e->lazy_ = true;
  return e;
}

std::shared_ptr<Event> Event::pending() {
  auto e = std::shared_ptr<Event>(new Event());
  e->pending_ = true;
  return e;
}

void Event::resolve(std::shared_ptr<Event> then) {
  {
    std::lock_guard<std::mutex> lk(mu_);
    if (!pending_) return;
    then_ = std::move(then);
    pending_ = false;
  }
  cv_.notify_all();
}

void Event::resolve_failed(Code code, const std::string& msg) {
  {
    std::lock_guard<std::mutex> lk(mu_);
    if (!pending_) return;
    pending_ = false;
    done_ = true;
    code_ = code;
    msg_ = msg;
  }
  cv_.notify_all();
}

void Event::wait_resolved() {
  std::unique_lock<std::mutex> lk(mu_);
  cv_.wait(lk, [&] { return !pending_; });
  if (done_ && code_ != Code::kOk) throw Error(code_, msg_);
}

bool Event::materialize_locked() {
  if (ev_ || !lazy_) return true;
  dev_->make_current();
  ev_ = dev_->take_event();
  const hipError_t r = hipEventRecord(ev_, dev_->stream());
  if (r != hipSuccess) {
    done_ = true;
    code_ = Code::kInternal;
    msg_ = std::string("hipEventRecord failed: ") + hipGetErrorString(r);
    return false;
  }
  return true;
}

Event::~Event() {
  if (!ev_) return;
  if (dev_) dev_->give_event(ev_);
  else (void)hipEventDestroy(ev_);
}

bool Event::is_ready() {
  std::unique_lock<std::mutex> lk(mu_);
  if (done_) return true;
  if (pending_) return false;
  if (then_) {
    std::shared_ptr<Event> t = then_;
    lk.unlock();
    const bool r = t->is_ready();
    lk.lock();
    if (r) {
      done_ = true;
      code_ = t->error_code();
      msg_ = t->error_message();
    }
    return done_;
  }
  if (lazy_ && !ev_) {
    // An idle stream has finished this work; otherwise record now.
    dev_->make_current();
    if (hipStreamQuery(dev_->stream()) == hipSuccess) {
      done_ = true;
      return true;
    }
    if (!materialize_locked()) return true;
  }
  hipError_t q = hipEventQuery(ev_);
  if (q == hipSuccess) {
    done_ = true;
  } else if (q != hipErrorNotReady) {
    done_ = true;
    code_ = Code::kInternal;
    msg_ = std::string("device work failed: ") + hipGetErrorString(q);
  }
  return done_;
}

void Event::await() {
  hipEvent_t ev = nullptr;
  {
    std::unique_lock<std::mutex> lk(mu_);
    cv_.wait(lk, [&] { return !pending_; });
    if (done_) return;
    if (then_) {
      std::shared_ptr<Event> t = then_;
      lk.unlock();
      t->await();
      lk.lock();
      done_ = true;
      code_ = t->error_code();
      msg_ = t->error_message();
      return;
    }
    if (!materialize_locked()) return;
    ev = ev_;
  }
  hipError_t e = hipEventSynchronize(ev);
  std::lock_guard<std::mutex> lk(mu_);
  done_ = true;
  if (e != hipSuccess) {
    code_ = Code::kInternal;
    msg_ = std::string("device work failed: ") + hipGetErrorString(e);
  }
}

void Event::on_ready(std::function<void()> fn) {
  if (is_ready()) {
    fn();
    return;
  }
  // The worker holds a reference until it has run the callback.
  EventWorker::get().push(shared_from_this(), std::move(fn));
}

// ------------------------------------------------------------------- buffers

BufferRef buffer_from_host(Device* dev, const TensorType& t, const void* data, const int64_t* byte_strides) {
  auto b = std::make_shared<Buffer>();
  b->dev = dev;
  b->type = t;
  const size_t bytes = t.bytes();
  b->mem = dev->allocate(bytes);
  if (bytes) {
    if (byte_strides) {
      // Dense row-major is required; reject other layouts explicitly.
      int64_t expect = static_cast<int64_t>(dtype_size(t.dtype));
      for (int d = t.rank() - 1; d >= 0; --d) {
        if (t.dims[d] != 1 && byte_strides[d] != expect)
          fail(Code::kUnimplemented, "BufferFromHostBuffer: only dense row-major host layouts are supported");
        expect *= t.dims[d];
      }
    }
    dev->make_current();
    if (staged_upload_wanted(bytes)) {
      staged_upload(dev, b->mem->ptr, data, bytes);
    } else {
      hip_check(hipMemcpyAsync(b->mem->ptr, data, bytes, hipMemcpyHostToDevice, dev->stream()), "hipMemcpyAsync(H2D)");
      hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize");
    }
  }
  b->ready = Event::ready();
  return b;
}

void buffer_to_host(const Buffer& b, void* dst, size_t dst_size) {
  const size_t bytes = b.type.bytes();
  PJRTX_CHECK(dst_size >= bytes, Code::kInvalidArgument,
              strformat("ToHostBuffer: destination holds %zu bytes, buffer needs %zu", dst_size, bytes));
  if (b.ready) b.ready->wait_resolved();  // an async transfer still filling it, or its error
  if (!bytes) return;
  if (staged_download_wanted(bytes)) {
    staged_download(b.dev, dst, b.mem->ptr, bytes);
    return;
  }
  b.dev->make_current();
  hip_check(hipMemcpyAsync(dst, b.mem->ptr, bytes, hipMemcpyDeviceToHost, b.dev->stream()), "hipMemcpyAsync(D2H)");
  hip_check(hipStreamSynchronize(b.dev->stream()), "hipStreamSynchronize");
}

// ------------------------------------------------------------ kernel compile

std::string kernel_translation_unit(const std::string& body) {
  return std::string(kFusionDeviceHeader) + "\n" + body;
}

namespace {
uint64_t fnv1a(const std::string& s, uint64_t seed) {
  uint64_t h = seed;
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

std::string cache_dir() {
  const char* d = std::getenv("PJRTX_KERNEL_CACHE_DIR");
  if (d && *d) return d;
  const char* home = std::getenv("HOME");
  return std::string(home ? home : "/tmp") + "/.cache/pjrtx_amd";
}

std::mutex g_compile_mu;
std::map<std::string, std::vector<char>> g_code_cache;
}  // namespace

std::vector<char> compile_kernels(const std::string& body, const std::string& arch) {
  const std::string src = kernel_translation_unit(body);
  const std::vector<std::string> opts = {
      "--offload-arch=" + arch, "-O3", "-std=c++17", "-ffp-contract=fast",
      // Packed f32 math is kept off: hand-written code relies on scalar f32.
      "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops"};
  std::string key_src = src;
  for (auto& o : opts) key_src += "\n//" + o;
  const std::string key = strformat("%016llx%016llx", static_cast<unsigned long long>(fnv1a(key_src, 1469598103934665603ull)),
                                    static_cast<unsigned long long>(fnv1a(key_src, 0x9e3779b97f4a7c15ull)));
  std::lock_guard<std::mutex> lk(g_compile_mu);
  auto it = g_code_cache.find(key);
  if (it != g_code_cache.end()) return it->second;
  const bool use_disk = !env_flag("PJRTX_NO_KERNEL_DISK_CACHE");
  const std::string path = cache_dir() + "/" + key + ".co";
  if (use_disk) {
    std::ifstream f(path, std::ios::binary);
    if (f) {
      std::vector<char> code((std::istreambuf_iterator<char>(f)), std::istreambuf_iterator<char>());
      if (!code.empty()) {
        g_code_cache[key] = code;
        return code;
      }
    }
  }
  hiprtcProgram prog;
  if (hiprtcCreateProgram(&prog, src.c_str(), "pjrtx_fusion.hip", 0, nullptr, nullptr) != HIPRTC_SUCCESS)
    fail(Code::kInternal, "hiprtcCreateProgram failed");
  std::vector<const char*> copts;
  for (auto& o : opts) copts.push_back(o.c_str());
  hiprtcResult r = hiprtcCompileProgram(prog, static_cast<int>(copts.size()), copts.data());
  size_t log_size = 0;
  hiprtcGetProgramLogSize(prog, &log_size);
  std::string log(log_size, '\0');
  if (log_size) hiprtcGetProgramLog(prog, log.data());
  if (r != HIPRTC_SUCCESS) {
    hiprtcDestroyProgram(&prog);
    if (env_flag("PJRTX_DUMP_KERNELS_ON_ERROR")) std::fprintf(stderr, "%s\n", src.c_str());
    fail(Code::kInternal, "hiprtc compile of fusion kernels failed:\n" + log.substr(0, 4000));
  }
  size_t code_size = 0;
  hiprtcGetCodeSize(prog, &code_size);
  std::vector<char> code(code_size);
  hiprtcGetCode(prog, code.data());
  hiprtcDestroyProgram(&prog);
  if (use_disk) {
    std::string dir = cache_dir();
    for (size_t pos = 1; pos != std::string::npos;) {
      pos = dir.find('/', pos + 1);
      ::mkdir(dir.substr(0, pos).c_str(), 0755);
    }
    const std::string tmp = path + strformat(".tmp%d", static_cast<int>(::getpid()));
    std::ofstream f(tmp, std::ios::binary);
    if (f) {
      f.write(code.data(), static_cast<std::streamsize>(code.size()));
      f.close();
      std::rename(tmp.c_str(), path.c_str());
    }
  }
  g_code_cache[key] = code;
  return code;
}

// ---------------------------------------------------------------- executable

namespace {

// A while's region as a program of its own: parameters are the loop state
// (the region's block arguments) then the captured values; results are the
// region's return operands.
Program region_program(const Program& prog, const Op& op, int which) {
  const Region& r = op.regions.at(which);
  Program sub;
  sub.module_name = prog.module_name + (which == 0 ? ".while_cond" : ".while_body");
  sub.values = prog.values;
  const size_t n_state = op.sizes.empty() ? op.operands.size() : static_cast<size_t>(op.sizes[0]);
  sub.params = r.params;
  for (size_t i = n_state; i < op.operands.size(); ++i) sub.params.push_back(op.operands[i]);
  // The body may write its state in place (a KV cache updated by a
  // dynamic_update_slice): the state blocks are donors, and run_while hands
  // the body only blocks the loop owns alone. Captured values and the
  // cond's arguments are never written.
  sub.param_alias.assign(sub.params.size(), -1);
  if (which == 1)
    for (size_t i = 0; i < n_state; ++i) sub.param_alias[i] = -2;
  for (const Op& o : r.ops) {
    if (o.kind == OpKind::kReturn) sub.results = o.operands;
    sub.ops.push_back(o);
  }
  PJRTX_CHECK(!sub.ops.empty() && sub.ops.back().kind == OpKind::kReturn, Code::kInvalidArgument,
              "while region does not end with a return");
  return sub;
}

MemRef copy_block(Device* dev, const MemRef& m) {
  MemRef c = dev->allocate(m->bytes);
  if (m->bytes)
    hip_check(hipMemcpyAsync(c->ptr, m->ptr, m->bytes, hipMemcpyDeviceToDevice, dev->stream()), "hipMemcpyAsync(D2D)");
  return c;
}

}  // namespace

Executable::Executable(Program prog, Plan plan, std::string fingerprint, std::string name)
    : prog_(std::move(prog)), plan_(std::move(plan)), fingerprint_(std::move(fingerprint)), name_(std::move(name)) {
  for (size_t si = 0; si < plan_.steps.size(); ++si) {
    const Step& s = plan_.steps[si];
    if (s.kind != StepKind::kLibrary || s.lib != LibKind::kWhile) continue;
    const Op& op = prog_.ops.at(s.lib_op);
    auto w = std::make_unique<WhileLoop>();
    for (int which = 0; which < 2; ++which) {
      Program sub = region_program(prog_, op, which);
      rewrite_program(&sub);
      Plan sp = make_plan(sub);
      auto e = std::make_unique<Executable>(std::move(sub), std::move(sp), fingerprint_, name_ + (which ? ".body" : ".cond"));
      (which == 0 ? w->cond : w->body) = std::move(e);
    }
    w->trips = s.while_trips;
    loops_[si] = std::move(w);
  }
}

int64_t Executable::while_trips(size_t si) const {
  auto it = loops_.find(si);
  return it == loops_.end() ? -1 : it->second->trips;
}

// ------------------------------------------------------------- residency

namespace {

struct ResidentEntry {
  Executable* exe = nullptr;
  int64_t bytes = 0;
  uint64_t last_use = 0;
  int busy = 0;
};

struct Residency {
  std::mutex mu;
  std::map<int, std::map<Executable*, ResidentEntry>> by_device;
  std::map<int, ResidencyStats> stats;
  uint64_t clock = 0;
};

Residency& residency() {
  static Residency* r = new Residency();
  return *r;
}

int64_t default_max_resident_bytes() { return env_int("PJRTX_MAX_RESIDENT_BYTES", 0); }

ResidencyStats& stats_locked(Residency& r, int ord) {
  auto it = r.stats.find(ord);
  if (it == r.stats.end()) {
    ResidencyStats st;
    st.max_resident_bytes = default_max_resident_bytes();
    it = r.stats.emplace(ord, st).first;
  }
  return it->second;
}

// Marks an executable busy on a device for a scope (not evictable).
class BusyScope {
 public:
  BusyScope(Executable* e, int ord) : e_(e), ord_(ord) {
    Residency& r = residency();
    std::lock_guard<std::mutex> lk(r.mu);
    ResidentEntry& en = r.by_device[ord][e];
    en.exe = e;
    en.busy++;
    en.last_use = ++r.clock;
  }
  ~BusyScope() {
    Residency& r = residency();
    std::lock_guard<std::mutex> lk(r.mu);
    auto d = r.by_device.find(ord_);
    if (d == r.by_device.end()) return;
    auto it = d->second.find(e_);
    if (it != d->second.end()) it->second.busy--;
  }

 private:
  Executable* e_;
  int ord_;
};

// Evicts idle executables (not `keep`) until `incoming` more bytes fit under
// the cap. Caller holds the device's execute lock, so no idle executable can
// start executing on this device meanwhile.
void make_room(int ord, Executable* keep, int64_t incoming) {
  std::vector<Executable*> victims;
  {
    Residency& r = residency();
    std::lock_guard<std::mutex> lk(r.mu);
    ResidencyStats& st = stats_locked(r, ord);
    if (st.max_resident_bytes <= 0) return;
    auto& entries = r.by_device[ord];
    int64_t total = st.resident_bytes;
    std::set<Executable*> chosen;
    while (total + incoming > st.max_resident_bytes) {
      const ResidentEntry* best = nullptr;
      for (auto& [e, en] : entries) {
        if (e == keep || en.busy > 0 || en.bytes <= 0 || chosen.count(e)) continue;
        if (!best || en.bytes > best->bytes || (en.bytes == best->bytes && en.last_use < best->last_use)) best = &en;
      }
      if (!best) break;  // everything left is busy: load past the cap
      total -= best->bytes;
      st.evictions++;
      st.evicted_bytes += best->bytes;
      chosen.insert(best->exe);
      victims.push_back(best->exe);
    }
  }
  for (Executable* e : victims) e->evict(ord);
}

void register_resident(int ord, Executable* e, int64_t bytes) {
  Residency& r = residency();
  std::lock_guard<std::mutex> lk(r.mu);
  ResidencyStats& st = stats_locked(r, ord);
  ResidentEntry& en = r.by_device[ord][e];
  en.exe = e;
  st.resident_bytes += bytes - en.bytes;
  if (en.bytes == 0) st.entries++;
  en.bytes = bytes;
  en.last_use = ++r.clock;
  st.peak_resident_bytes = std::max(st.peak_resident_bytes, st.resident_bytes);
}

// Takes an executable's bytes on a device out of the total; `erase` also
// forgets the entry (the executable is being destroyed).
void unregister_resident(int ord, Executable* e, bool erase) {
  Residency& r = residency();
  std::lock_guard<std::mutex> lk(r.mu);
  auto d = r.by_device.find(ord);
  if (d == r.by_device.end()) return;
  auto it = d->second.find(e);
  if (it == d->second.end()) return;
  ResidencyStats& st = stats_locked(r, ord);
  if (it->second.bytes > 0) {
    st.resident_bytes -= it->second.bytes;
    st.entries--;
  }
  it->second.bytes = 0;
  if (erase) d->second.erase(it);
}

// Drops every device's entry for a destroyed executable.
void forget_resident(Executable* e) {
  Residency& r = residency();
  std::lock_guard<std::mutex> lk(r.mu);
  for (auto& [ord, entries] : r.by_device) {
    auto it = entries.find(e);
    if (it == entries.end()) continue;
    ResidencyStats& st = stats_locked(r, ord);
    if (it->second.bytes > 0) {
      st.resident_bytes -= it->second.bytes;
      st.entries--;
    }
    entries.erase(it);
  }
}

}  // namespace

ResidencyStats residency_stats(int ordinal) {
  Residency& r = residency();
  std::lock_guard<std::mutex> lk(r.mu);
  return stats_locked(r, ordinal);
}

void set_max_resident_bytes(int ordinal, int64_t bytes) {
  Residency& r = residency();
  std::lock_guard<std::mutex> lk(r.mu);
  stats_locked(r, ordinal).max_resident_bytes = std::max<int64_t>(0, bytes);
}

std::vector<MemRef> Executable::run_values(Device* dev, const std::vector<MemRef>& args) {
  PJRTX_CHECK(args.size() == prog_.params.size(), Code::kInternal, "run_values: argument count");
  BusyScope busy(this, dev->ordinal());
  Loaded* L = loaded_for(dev, true);
  std::vector<MemRef> vals(prog_.values.size());
  for (size_t i = 0; i < args.size(); ++i) vals[prog_.params[i]] = args[i];
  for (auto& [v, m] : L->constants) vals[v] = m;
  for (size_t si = 0; si < plan_.steps.size(); ++si) {
    run_step(L, si, vals);
    for (int v : plan_.steps[si].release_after) vals[v].reset();
  }
  std::vector<MemRef> out;
  for (int r : prog_.results) {
    PJRTX_CHECK(vals[r] != nullptr, Code::kInternal, "run_values: result value was not produced");
    out.push_back(vals[r]);
  }
  return out;
}

// Runs a while step: the loop state lives in device blocks the loop owns.
// With a constant-fixed count the body runs that many times back to back
// (no host round trip); otherwise each iteration runs the cond, reads its
// predicate on the host and stops when it is false (the reference's
// general while: execution_control_flow_while.zig, which only runs a
// recognised f32 counter pattern on the device).
void Executable::run_while(Loaded* L, size_t si, std::vector<MemRef>& vals) {
  Device* dev = L->dev;
  const Step& s = plan_.steps[si];
  const Op& op = prog_.ops.at(s.lib_op);
  WhileLoop& w = *loops_.at(si);
  const size_t n = static_cast<size_t>(op.sizes.at(0));
  std::vector<MemRef> state(n), caps;
  for (size_t i = 0; i < n; ++i) state[i] = vals[op.operands[i]];
  for (size_t i = n; i < op.operands.size(); ++i) caps.push_back(vals[op.operands[i]]);
  auto args_for = [&](const Executable& region) {
    std::vector<MemRef> a = state;
    a.insert(a.end(), caps.begin(), caps.end());
    // A captured value the region writes in place is the caller's, and the
    // cond must not change the state: those get copies.
    for (int k : region.plan().written_params)
      if ((static_cast<size_t>(k) >= n || &region == w.cond.get()) && a[k]) a[k] = copy_block(dev, a[k]);
    return a;
  };
  // The body writes these state blocks in place: each must be the loop's
  // alone (not the caller's value, a constant or another state slot).
  auto own_written = [&]() {
    for (int k : w.body->plan().written_params)
      if (static_cast<size_t>(k) < n && state[k] && state[k].use_count() > 1) state[k] = copy_block(dev, state[k]);
  };
  auto run_body = [&]() {
    own_written();
    std::vector<MemRef> next = w.body->run_values(dev, args_for(*w.body));
    PJRTX_CHECK(next.size() == n, Code::kInternal, "while body returned the wrong number of values");
    state = std::move(next);
  };
  if (w.trips >= 0) {
    for (int64_t t = 0; t < w.trips; ++t) run_body();
  } else {
    for (;;) {
      std::vector<MemRef> pred = w.cond->run_values(dev, args_for(*w.cond));
      PJRTX_CHECK(pred.size() == 1 && pred[0]->bytes >= 1, Code::kInternal, "while cond must return one predicate");
      uint8_t go = 0;
      hip_check(hipMemcpyAsync(&go, pred[0]->ptr, 1, hipMemcpyDeviceToHost, dev->stream()), "hipMemcpyAsync(pred)");
      hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize");
      if (!go) break;
      run_body();
    }
  }
  // A result that is still one of the operands' blocks (a passed-through
  // state element, or no iteration at all) gets its own copy.
  for (size_t i = 0; i < n; ++i) {
    bool shared = false;
    for (int v : op.operands) shared = shared || (vals[v] && vals[v].get() == state[i].get());
    vals[op.results[i]] = shared ? copy_block(dev, state[i]) : state[i];
  }
  stats_.library_calls++;
}

void Executable::evict(int ordinal) {
  std::unique_ptr<Loaded> gone;
  {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = loaded_.find(ordinal);
    if (it != loaded_.end()) {
      gone = std::move(it->second);
      loaded_.erase(it);
    }
  }
  if (gone) {
    // Kernels and graphs this executable queued may still run: drain the
    // device's stream before the graphs, the module and its memory go.
    gone->dev->make_current();
    hip_check(hipStreamSynchronize(gone->dev->stream()), "hipStreamSynchronize(evict)");
  }
  {
    std::lock_guard<std::mutex> lk(mu_);
    graphs_.erase(ordinal);
  }
  if (gone && gone->module) (void)hipModuleUnload(gone->module);
  for (auto& [si, loop] : loops_) {
    if (loop->cond) loop->cond->evict(ordinal);
    if (loop->body) loop->body->evict(ordinal);
  }
  unregister_resident(ordinal, this, false);
}

Executable::~Executable() {
  for (auto& [ord, L] : loaded_) {
    if (L->module) (void)hipModuleUnload(L->module);
  }
  forget_resident(this);
}

void Executable::load(Device* dev) {
  std::lock_guard<std::mutex> lk(dev->exec_mutex());
  BusyScope busy(this, dev->ordinal());
  loaded_for(dev, true);
}

Executable::Loaded* Executable::loaded_for(Device* dev, bool may_evict) {
  {
    std::lock_guard<std::mutex> lk(mu_);
    auto it = loaded_.find(dev->ordinal());
    if (it != loaded_.end()) return it->second.get();
  }
  if (may_evict) {
    int64_t incoming = static_cast<int64_t>(code_.size());
    for (const Step& st : plan_.steps) incoming += static_cast<int64_t>(st.scratch_bytes);
    for (int v : plan_.constants) incoming += prog_.type(v).bytes();
    make_room(dev->ordinal(), this, incoming);
  }
  std::lock_guard<std::mutex> lk(mu_);
  auto it = loaded_.find(dev->ordinal());
  if (it != loaded_.end()) return it->second.get();
  auto L = std::make_unique<Loaded>();
  L->dev = dev;
  dev->make_current();
  if (plan_.num_fusion_kernels > 0) {
    if (code_.empty()) code_ = compile_kernels(plan_.kernel_source, dev->arch());
    hip_check(hipModuleLoadData(&L->module, code_.data()), "hipModuleLoadData");
  }
  L->funcs.resize(plan_.steps.size(), nullptr);
  L->combine_funcs.resize(plan_.steps.size(), nullptr);
  L->scratch.resize(plan_.steps.size());
  for (size_t i = 0; i < plan_.steps.size(); ++i) {
    const Step& s = plan_.steps[i];
    if (s.kind == StepKind::kLoop || s.kind == StepKind::kReduce || s.kind == StepKind::kRowFused ||
        s.kind == StepKind::kGemv) {
      hip_check(hipModuleGetFunction(&L->funcs[i], L->module, s.name.c_str()), "hipModuleGetFunction");
    }
    if (s.combine_grid) {
      const std::string cname = s.name + "_combine";
      hip_check(hipModuleGetFunction(&L->combine_funcs[i], L->module, cname.c_str()), "hipModuleGetFunction");
    }
    if (s.scratch_bytes) L->scratch[i] = dev->allocate(s.scratch_bytes);
    if (s.fused_combine) {
      // Arrival counters start at zero; the last workgroup of each row puts
      // its row's counter back to zero, so every later launch (and graph
      // replay) finds them cleared without a memset in the execute path.
      uint8_t* ctr = static_cast<uint8_t*>(L->scratch[i]->ptr) + s.counter_offset;
      hip_check(hipMemsetAsync(ctr, 0, s.scratch_bytes - s.counter_offset, dev->stream()), "hipMemsetAsync(counters)");
      hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize");
    }
  }
  // Resident constants: uploaded once (reference: executable_constants.zig:32-83).
  for (int v : plan_.constants) {
    int oi = plan_.producer.at(v);
    const Op& op = prog_.ops[oi];
    const TensorType& t = prog_.type(v);
    std::vector<uint8_t> full;
    const uint8_t* src = op.literal.data();
    if (op.splat) {
      const size_t esz = dtype_size(t.dtype);
      full.resize(t.bytes());
      for (int64_t k = 0; k < t.elements(); ++k) std::memcpy(full.data() + k * esz, op.literal.data(), esz);
      src = full.data();
    }
    MemRef m = dev->allocate(t.bytes());
    // Stream-ordered upload: the block may have been freed by work still
    // queued on this stream.
    if (t.bytes()) {
      hip_check(hipMemcpyAsync(m->ptr, src, t.bytes(), hipMemcpyHostToDevice, dev->stream()), "hipMemcpyAsync(constant)");
      hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize");
    }
    L->constants[v] = m;
  }
  hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize");
  Loaded* raw = L.get();
  int64_t resident = static_cast<int64_t>(code_.size());
  for (const MemRef& m : L->scratch)
    if (m) resident += static_cast<int64_t>(m->bytes);
  for (auto& [v, m] : L->constants)
    if (m) resident += static_cast<int64_t>(m->bytes);
  loaded_[dev->ordinal()] = std::move(L);
  register_resident(dev->ordinal(), this, resident);
  return raw;
}

void Executable::run_step(Loaded* L, size_t si, std::vector<MemRef>& vals, int phase) {
  const Step& s = plan_.steps[si];
  Device* dev = L->dev;
  switch (s.kind) {
    case StepKind::kAlias:
      vals[s.outputs[0]] = vals[s.inputs[0]];
      return;
    case StepKind::kLibrary:
      if (s.lib == LibKind::kWhile) {
        run_while(L, si, vals);
        return;
      }
      if (s.in_place) {
        vals[s.outputs[0]] = vals[prog_.ops[s.lib_op].operands[0]];
      } else if (s.attn_partials) {
        vals[s.outputs[0]] = dev->allocate(attention_partials_bytes(prog_, prog_.ops[s.lib_op]));
      } else {
        for (int v : s.outputs) vals[v] = dev->allocate(prog_.type(v).bytes());
      }
      run_library_step(dev, prog_, s, vals);
      stats_.library_calls++;
      return;
    case StepKind::kLoop:
    case StepKind::kReduce:
    case StepKind::kRowFused:
    case StepKind::kGemv: {
      if (phase != 1) {
        for (size_t k = 0; k < s.outputs.size(); ++k) {
          auto ww = s.window_out.find(static_cast<int>(k));
          // A fused in-place dynamic_update_slice result is its operand's buffer.
          vals[s.outputs[k]] = ww != s.window_out.end() ? vals[ww->second.operand]
                                                        : dev->allocate(prog_.type(s.outputs[k]).bytes());
        }
      }
      if (s.kind == StepKind::kLoop && num_elements(s.loop_shape) == 0) return;
      if ((s.kind == StepKind::kReduce || s.kind == StepKind::kRowFused) && s.rows == 0) return;
      std::vector<void*> ptrs;
      ptrs.reserve(s.inputs.size() + s.outputs.size() + 2);
      for (int v : s.inputs) ptrs.push_back(vals[v] ? vals[v]->ptr : nullptr);
      for (int v : s.outputs) ptrs.push_back(vals[v]->ptr);
      MemRef arena_scratch;
      // A fused combine folds the partials inside the main launch when the
      // device places workgroups round-robin on its XCDs; otherwise the
      // `_combine` kernel runs after it.
      const uint32_t fused_mode = s.fused_combine && dev->xcd_round_robin() ? 1u : 0u;
      if (s.scratch_bytes && thread_arena() && phase != 1) {
        // Allocation-free execute: partial slots from the fixed block; the
        // arrival counters of a one-launch fold must start at zero.
        arena_scratch = dev->allocate(s.scratch_bytes);
        if (s.fused_combine) {
          const size_t lo = s.counter_offset & ~size_t(15);
          const size_t hi = (s.scratch_bytes + 15) & ~size_t(15);
          launch_noalloc_zero(dev->stream(), static_cast<uint8_t*>(arena_scratch->ptr) + lo, hi - lo);
        }
        ptrs.push_back(arena_scratch->ptr);
      } else if (s.scratch_bytes) {
        ptrs.push_back(L->scratch[si]->ptr);
      }
      std::vector<void*> args(ptrs.size());
      for (size_t k = 0; k < ptrs.size(); ++k) args[k] = &ptrs[k];
      if (s.fused_combine) args.push_back(const_cast<uint32_t*>(&fused_mode));
      if (phase != 1) {
        hip_check(hipModuleLaunchKernel(L->funcs[si], s.grid, 1, 1, s.block, 1, 1, 0, dev->stream(), args.data(),
                                        nullptr),
                  "hipModuleLaunchKernel");
        stats_.kernel_launches++;
      }
      if (s.combine_grid && phase != 0 && !fused_mode) {
        // Second pass of a split reduction: same arguments, one wave per row.
        hip_check(hipModuleLaunchKernel(L->combine_funcs[si], s.combine_grid, 1, 1, 256, 1, 1, 0, dev->stream(),
                                        args.data(), nullptr),
                  "hipModuleLaunchKernel(combine)");
        stats_.kernel_launches++;
      }
      return;
    }
  }
}

std::vector<BufferRef> Executable::execute(Device* dev, const std::vector<BufferRef>& args,
                                           std::shared_ptr<Event>* done, const std::vector<bool>* donate) {
  PJRTX_CHECK(args.size() == prog_.params.size(), Code::kInvalidArgument,
              strformat("execute: program takes %zu arguments, got %zu", prog_.params.size(), args.size()));
  for (size_t i = 0; i < args.size(); ++i) {
    const TensorType& want = prog_.type(prog_.params[i]);
    PJRTX_CHECK(args[i] && !args[i]->deleted, Code::kInvalidArgument, strformat("execute: argument %zu is deleted", i));
    PJRTX_CHECK(args[i]->type == want, Code::kInvalidArgument,
                strformat("execute: argument %zu has type %s, program expects %s", i, args[i]->type.str().c_str(),
                          want.str().c_str()));
    PJRTX_CHECK(args[i]->dev == dev, Code::kInvalidArgument, strformat("execute: argument %zu is on another device", i));
    // An argument still receiving an async host transfer: wait for its last
    // chunk (the chunks are queued on this device's stream, ahead of us).
    if (args[i]->ready) args[i]->ready->wait_resolved();
  }
  std::lock_guard<std::mutex> lk(dev->exec_mutex());
  BusyScope busy(this, dev->ordinal());
  Loaded* L = loaded_for(dev, true);
  dev->make_current();
  // Repeated executions with the same large arguments replay a captured
  // graph (second call captures, later calls replay).
  if (graph_candidate(args, donate)) {
    GraphState& gs = graph_state(dev->ordinal());
    std::vector<const void*> key = graph_key(args);
    for (auto& e : gs.entries)
      if (e->key == key) return replay_graph(dev, e.get(), args, done);
    bool seen_before = false;
    for (auto& k : gs.seen) seen_before = seen_before || k == key;
    if (seen_before) {
      GraphEntry* g = capture_graph(dev, L, args, key);
      if (g) return replay_graph(dev, g, args, done);
    } else {
      gs.seen.push_back(key);
      if (gs.seen.size() > 8) gs.seen.erase(gs.seen.begin());
    }
  }
  std::vector<MemRef> vals(prog_.values.size());
  for (size_t i = 0; i < args.size(); ++i) vals[prog_.params[i]] = args[i]->mem;
  auto donated = [&](size_t i) { return donate && i < donate->size() && (*donate)[i]; };
  for (int k : plan_.written_params) {
    if (donated(k)) continue;
    // The plan writes this parameter in place; keep the caller's buffer intact.
    const MemRef& src = args[k]->mem;
    MemRef c = dev->allocate(src->bytes);
    if (src->bytes)
      hip_check(hipMemcpyAsync(c->ptr, src->ptr, src->bytes, hipMemcpyDeviceToDevice, dev->stream()),
                "hipMemcpyAsync(undonated argument)");
    vals[prog_.params[k]] = c;
  }
  for (auto& [v, m] : L->constants) vals[v] = m;
  for (size_t si = 0; si < plan_.steps.size(); ++si) {
    run_step(L, si, vals);
    for (int v : plan_.steps[si].release_after) {
      vals[v].reset();
      stats_.released_values++;
    }
  }
  // Outputs: a result that is an argument, a constant or repeated gets its
  // own copy so that every returned buffer owns distinct memory.
  std::vector<BufferRef> outs;
  std::set<const DeviceMemory*> seen;
  std::set<const DeviceMemory*> borrowed;
  for (size_t i = 0; i < args.size(); ++i)
    if (!donated(i)) borrowed.insert(args[i]->mem.get());
  for (auto& [v, m] : L->constants) borrowed.insert(m.get());
  for (int r : prog_.results) {
    MemRef m = vals[r];
    PJRTX_CHECK(m != nullptr, Code::kInternal, "execute: result value was not produced");
    if (borrowed.count(m.get()) || seen.count(m.get())) {
      MemRef c = dev->allocate(m->bytes);
      if (m->bytes)
        hip_check(hipMemcpyAsync(c->ptr, m->ptr, m->bytes, hipMemcpyDeviceToDevice, dev->stream()), "hipMemcpyAsync(D2D)");
      m = c;
    }
    seen.insert(m.get());
    auto b = std::make_shared<Buffer>();
    b->dev = dev;
    b->type = prog_.type(r);
    b->mem = m;
    outs.push_back(b);
  }
  std::shared_ptr<Event> ev = Event::record(dev);
  for (auto& b : outs) b->ready = ev;
  if (done) *done = ev;
  stats_.executions++;
  return outs;
}

size_t Executable::execute_noalloc(Device* dev, const void* const* args, size_t num_args, void* const* outs,
                                   size_t num_outs) {
  PJRTX_CHECK(num_args == prog_.params.size(), Code::kInvalidArgument,
              strformat("execute_noalloc: program takes %zu arguments, got %zu", prog_.params.size(), num_args));
  PJRTX_CHECK(num_outs == prog_.results.size(), Code::kInvalidArgument,
              strformat("execute_noalloc: program has %zu results, got %zu output pointers", prog_.results.size(),
                        num_outs));
  PJRTX_CHECK(loops_.empty(), Code::kUnimplemented,
              "execute_noalloc: programs with a while loop are not supported (their regions load on first use)");
  for (size_t i = 0; i < num_args; ++i)
    PJRTX_CHECK(args[i] || prog_.type(prog_.params[i]).bytes() == 0, Code::kInvalidArgument,
                strformat("execute_noalloc: argument %zu is null", i));
  for (size_t i = 0; i < num_outs; ++i)
    PJRTX_CHECK(outs[i] || prog_.type(prog_.results[i]).bytes() == 0, Code::kInvalidArgument,
                strformat("execute_noalloc: output %zu is null", i));
  // Same order as execute(): the device's execute lock first, then busy (so
  // no other thread's load can evict this executable while it runs; busy
  // also refreshes its last use for the residency budget), then the lookup.
  std::lock_guard<std::mutex> lk(dev->exec_mutex());
  BusyScope busy(this, dev->ordinal());
  Loaded* L = nullptr;
  {
    std::lock_guard<std::mutex> lk2(mu_);
    auto it = loaded_.find(dev->ordinal());
    PJRTX_CHECK(it != loaded_.end(), Code::kFailedPrecondition,
                strformat("execute_noalloc: the executable is not loaded on device %d (loading allocates)",
                          dev->ordinal()));
    L = it->second.get();
  }
  dev->make_current();
  Arena arena;
  arena.dev = dev;
  arena.base = static_cast<uint8_t*>(noalloc_scratch(dev->ordinal()));
  arena.cap = kNoallocScratchBytes;
  ArenaScope scope(&arena);
  std::vector<MemRef> vals(prog_.values.size());
  for (size_t i = 0; i < num_args; ++i) {
    auto m = std::make_shared<DeviceMemory>();
    m->dev = dev;
    m->ptr = const_cast<void*>(args[i]);
    m->bytes = prog_.type(prog_.params[i]).bytes();
    m->capacity = m->bytes;
    m->borrowed = true;
    vals[prog_.params[i]] = m;
  }
  for (int k : plan_.written_params) {
    // The plan writes this parameter in place: work on a copy, the caller's
    // input stays as it was.
    const MemRef& src = vals[prog_.params[k]];
    MemRef c = dev->allocate(src->bytes);
    if (src->bytes)
      hip_check(hipMemcpyAsync(c->ptr, src->ptr, src->bytes, hipMemcpyDeviceToDevice, dev->stream()),
                "hipMemcpyAsync(written argument)");
    vals[prog_.params[k]] = c;
  }
  for (auto& [v, m] : L->constants) vals[v] = m;
  for (size_t si = 0; si < plan_.steps.size(); ++si) {
    run_step(L, si, vals);
    for (int v : plan_.steps[si].release_after) vals[v].reset();
  }
  for (size_t i = 0; i < num_outs; ++i) {
    const MemRef& m = vals[prog_.results[i]];
    PJRTX_CHECK(m != nullptr, Code::kInternal, "execute_noalloc: result value was not produced");
    if (m->bytes && m->ptr != outs[i])
      hip_check(hipMemcpyAsync(outs[i], m->ptr, m->bytes, hipMemcpyDeviceToDevice, dev->stream()),
                "hipMemcpyAsync(result)");
  }
  stats_.executions++;
  return arena.peak;
}

// ------------------------------------------------------------ graph replay

namespace {
constexpr size_t kGraphStagedMaxBytes = 64 * 1024;   // arguments up to this size are copied in
constexpr size_t kGraphMaxPinnedBytes = 256u << 20;  // graphs holding more memory are not kept
constexpr size_t kGraphEntriesPerDevice = 4;
constexpr int kGraphMinLaunches = 8;
// Mean bytes a launch moves below which a plan is launch-bound (its kernels
// take about as long as the host needs to launch them), so that replaying
// it from a graph pays for the graph's staging copies. Heavier plans keep
// the GPU busy from eager launches alone (the llama-like decode step: 46
// launches of 21 MB on average runs 4% faster eager).
constexpr double kGraphLaunchBoundBytes = 4.0 * (1 << 20);
}  // namespace

Executable::GraphState& Executable::graph_state(int ordinal) {
  std::lock_guard<std::mutex> lk(mu_);
  return graphs_[ordinal];  // std::map: references stay valid
}

Executable::GraphEntry::~GraphEntry() {
  if (exec) (void)hipGraphExecDestroy(exec);
}

bool Executable::graph_candidate(const std::vector<BufferRef>& args, const std::vector<bool>* donate) const {
  // PJRTX_GRAPHS: 0 never, 1 (default) launch-bound plans, 2 every plan.
  const int64_t mode = env_int("PJRTX_GRAPHS", 1);
  if (mode == 0) return false;
  if (!loops_.empty()) return false;  // a while reads its predicate on the host
  if (mode == 1) {
    double bytes = 0;
    int n = 0;
    for (const Step& st : plan_.steps) {
      if (st.kind == StepKind::kAlias) continue;
      ++n;
      for (int v : st.inputs) bytes += static_cast<double>(prog_.type(v).bytes());
      for (size_t k = 0; k < st.outputs.size(); ++k) {
        auto ww = st.window_out.find(static_cast<int>(k));
        bytes += static_cast<double>(prog_.type(ww == st.window_out.end() ? st.outputs[k] : ww->second.update).bytes());
      }
    }
    if (n == 0 || bytes / n >= kGraphLaunchBoundBytes) return false;
  }
  if (args.empty() || const_cast<Executable*>(this)->graph_state(args[0]->dev->ordinal()).disabled) return false;
  int launches = 0;
  for (const Step& st : plan_.steps) launches += st.kind != StepKind::kAlias;
  if (launches < kGraphMinLaunches) return false;
  for (int k : plan_.written_params)  // in-place writes need the caller's donation
    if (!donate || static_cast<size_t>(k) >= donate->size() || !(*donate)[k]) return false;
  return true;
}

std::vector<const void*> Executable::graph_key(const std::vector<BufferRef>& args) const {
  std::set<int> written(plan_.written_params.begin(), plan_.written_params.end());
  std::vector<const void*> key(args.size(), nullptr);
  for (size_t i = 0; i < args.size(); ++i) {
    const bool staged = args[i]->mem->bytes <= kGraphStagedMaxBytes && !written.count(static_cast<int>(i));
    if (!staged) key[i] = args[i]->mem->ptr;
  }
  return key;
}

Executable::GraphEntry* Executable::capture_graph(Device* dev, Loaded* L, const std::vector<BufferRef>& args,
                                                  std::vector<const void*> key) {
  GraphState& gs = graph_state(dev->ordinal());
  auto g = std::make_unique<GraphEntry>();
  g->key = std::move(key);
  dev->set_capture_pins(&g->pins);
  g->staging.resize(args.size());
  std::vector<MemRef> vals(prog_.values.size());
  for (size_t i = 0; i < args.size(); ++i) {
    if (g->key[i] == nullptr) {
      g->staging[i] = dev->allocate(args[i]->mem->bytes);
      vals[prog_.params[i]] = g->staging[i];
    } else {
      vals[prog_.params[i]] = args[i]->mem;
    }
  }
  for (auto& [v, m] : L->constants) vals[v] = m;
  hipGraph_t graph = nullptr;
  bool ok = hipStreamBeginCapture(dev->stream(), hipStreamCaptureModeRelaxed) == hipSuccess;
  if (ok) {
    try {
      for (size_t si = 0; si < plan_.steps.size(); ++si) run_step(L, si, vals);
    } catch (const std::exception&) {
      ok = false;
    }
    hipError_t e = hipStreamEndCapture(dev->stream(), &graph);
    ok = ok && e == hipSuccess && graph != nullptr;
  }
  (void)hipGetLastError();
  dev->set_capture_pins(nullptr);
  // Results must be graph-produced or donated argument memory, each distinct.
  std::set<const DeviceMemory*> pinned, seen;
  for (auto& m : g->pins) pinned.insert(m.get());
  for (int r : prog_.results) {
    if (!ok) break;
    const MemRef& m = vals[r];
    int param = -1;
    for (size_t i = 0; i < args.size() && param < 0; ++i)
      if (g->key[i] != nullptr && m.get() == args[i]->mem.get()) param = static_cast<int>(i);
    const bool internal = m && pinned.count(m.get());
    if (!m || seen.count(m.get()) || (param < 0 && !internal)) ok = false;
    if (param >= 0) {  // only donated (written-in-place) arguments may come back as results
      bool written = false;
      for (int k : plan_.written_params) written = written || k == param;
      if (!written) ok = false;
    }
    seen.insert(m.get());
    g->result_param.push_back(param);
    g->result_mem.push_back(param < 0 ? m : MemRef());
  }
  size_t pinned_bytes = 0;
  for (auto& m : g->pins) pinned_bytes += m->capacity;
  if (ok) ok = pinned_bytes <= kGraphMaxPinnedBytes;
  if (ok) ok = hipGraphInstantiate(&g->exec, graph, nullptr, nullptr, 0) == hipSuccess;
  if (graph) (void)hipGraphDestroy(graph);
  (void)hipGetLastError();
  if (!ok) {
    gs.disabled = true;  // run this executable eagerly from now on
    return nullptr;
  }
  stats_.graph_captures++;
  if (gs.entries.size() >= kGraphEntriesPerDevice) {
    auto lru = std::min_element(gs.entries.begin(), gs.entries.end(),
                                [](const auto& a, const auto& b) { return a->last_use < b->last_use; });
    // Its graph may still be queued: drain the stream before the executable
    // graph is destroyed (its blocks alone would be safe to hand back, since
    // reuse is ordered on the one stream).
    hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize(graph evict)");
    gs.entries.erase(lru);
  }
  gs.entries.push_back(std::move(g));
  return gs.entries.back().get();
}

std::vector<BufferRef> Executable::replay_graph(Device* dev, GraphEntry* g, const std::vector<BufferRef>& args,
                                                std::shared_ptr<Event>* done) {
  GraphState& gs = graph_state(dev->ordinal());
  g->last_use = ++gs.clock;
  CopySegments in;
  for (size_t i = 0; i < args.size(); ++i) {
    if (g->key[i] != nullptr || !args[i]->mem->bytes) continue;
    if (in.n == kMaxCopySegments) {
      launch_copy_segments(dev->stream(), in);
      in = CopySegments();
    }
    in.src[in.n] = args[i]->mem->ptr;
    in.dst[in.n] = g->staging[i]->ptr;
    in.bytes[in.n] = static_cast<int64_t>(args[i]->mem->bytes);
    in.n++;
  }
  launch_copy_segments(dev->stream(), in);
  hip_check(hipGraphLaunch(g->exec, dev->stream()), "hipGraphLaunch");
  std::vector<BufferRef> outs;
  CopySegments out;
  for (size_t r = 0; r < prog_.results.size(); ++r) {
    auto b = std::make_shared<Buffer>();
    b->dev = dev;
    b->type = prog_.type(prog_.results[r]);
    if (g->result_param[r] >= 0) {
      b->mem = args[g->result_param[r]]->mem;
    } else {
      const MemRef& src = g->result_mem[r];
      b->mem = dev->allocate(src->bytes);
      if (src->bytes) {
        if (out.n == kMaxCopySegments) {
          launch_copy_segments(dev->stream(), out);
          out = CopySegments();
        }
        out.src[out.n] = src->ptr;
        out.dst[out.n] = b->mem->ptr;
        out.bytes[out.n] = static_cast<int64_t>(src->bytes);
        out.n++;
      }
    }
    outs.push_back(b);
  }
  launch_copy_segments(dev->stream(), out);
  std::shared_ptr<Event> ev = Event::record(dev);
  for (auto& b : outs) b->ready = ev;
  if (done) *done = ev;
  stats_.executions++;
  stats_.graph_replays++;
  return outs;
}

std::vector<std::string> Executable::unit_names() const {
  std::vector<std::string> out;
  for (const Step& st : plan_.steps) {
    if (st.kind == StepKind::kLibrary) {
      out.push_back(std::string("lib:") + lib_kind_name(st.lib));
    } else if (st.kind == StepKind::kAlias) {
      out.push_back("-");
    } else {
      out.push_back(st.name);
      if (st.combine_grid && !st.fused_combine) out.push_back(st.name + "_combine");
    }
  }
  return out;
}

std::vector<double> Executable::time_steps(Device* dev, const std::vector<BufferRef>& args, int iters) {
  std::lock_guard<std::mutex> lk(dev->exec_mutex());
  BusyScope busy(this, dev->ordinal());
  Loaded* L = loaded_for(dev, true);
  dev->make_current();
  std::vector<MemRef> vals(prog_.values.size());
  for (size_t i = 0; i < args.size(); ++i) vals[prog_.params[i]] = args[i]->mem;
  for (auto& [v, m] : L->constants) vals[v] = m;
  std::vector<double> ms;
  hipEvent_t a, b;
  hip_check(hipEventCreate(&a), "hipEventCreate");
  hip_check(hipEventCreate(&b), "hipEventCreate");
  auto timed = [&](size_t si, int phase) {
    hip_check(hipEventRecord(a, dev->stream()), "hipEventRecord");
    for (int k = 0; k < iters; ++k) run_step(L, si, vals, phase);
    hip_check(hipEventRecord(b, dev->stream()), "hipEventRecord");
    hip_check(hipEventSynchronize(b), "hipEventSynchronize");
    float t = 0.f;
    hip_check(hipEventElapsedTime(&t, a, b), "hipEventElapsedTime");
    ms.push_back(static_cast<double>(t) / iters);
  };
  for (size_t si = 0; si < plan_.steps.size(); ++si) {
    const Step& st = plan_.steps[si];
    run_step(L, si, vals);  // warm and produce outputs for later steps
    bool split = st.kind != StepKind::kLibrary && st.kind != StepKind::kAlias && st.combine_grid && !st.fused_combine;
    if (split) {
      timed(si, 0);
      timed(si, 1);
    } else {
      timed(si, -1);
    }
  }
  (void)hipEventDestroy(a);
  (void)hipEventDestroy(b);
  return ms;
}

}  // namespace pjrtx
