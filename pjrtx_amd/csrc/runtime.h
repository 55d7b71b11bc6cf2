// Device runtime of the plugin: one HIP stream per GPU, a caching device
// allocator, readiness events, device-resident buffers, and the executable
// that replays a Plan as kernel launches.
//
// Replaces the reference's backend execute path
// (reference: src/backend/mlx_metal/execution_call.zig:66-145,
// execution_schedule.zig:58-197, execution_liveness.zig:16-52,
// metalcpp_api.cc:961-1161 value-table executor) and its buffer / event
// runtime (src/runtime/event.zig:30-95, src/runtime/execution_call.zig:39-102,
// api.cc:1781-1852 H2D, api.cc:5685-5731 D2H).
#pragma once

#include <hip/hip_runtime.h>

#include <atomic>
#include <condition_variable>
#include <deque>
#include <functional>
#include <map>
#include <memory>
#include <mutex>
#include <string>
#include <thread>
#include <vector>

#include "ir.h"
#include "planner.h"

namespace pjrtx {

void hip_check(hipError_t e, const char* what);

class Device;

// One block from the caching allocator; returned to the cache when the last
// reference drops. Reuse is stream-ordered because all work on a device is
// issued to its single stream.
struct DeviceMemory {
  Device* dev = nullptr;
  void* ptr = nullptr;
  size_t bytes = 0;     // requested
  size_t capacity = 0;  // allocated
  bool borrowed = false;  // not the allocator's (an arena block or caller memory): never released
  ~DeviceMemory();
};
using MemRef = std::shared_ptr<DeviceMemory>;

// A fixed device block that Device::allocate carves blocks from (bump order,
// 256-byte aligned) instead of calling the caching allocator, while it is
// installed on the calling thread for its device. Blocks are never handed
// back one by one: the next call that installs the arena starts at zero.
// Used by the allocation-free execute; exceeding `cap` fails with
// RESOURCE_EXHAUSTED.
struct Arena {
  Device* dev = nullptr;
  uint8_t* base = nullptr;
  size_t cap = 0;
  size_t used = 0;
  size_t peak = 0;
};
Arena* thread_arena();
class ArenaScope {
 public:
  explicit ArenaScope(Arena* a);
  ~ArenaScope();

 private:
  Arena* prev_;
};

class Allocator {
 public:
  explicit Allocator(int ordinal) : ordinal_(ordinal) {}
  ~Allocator();
  void* alloc(size_t bytes, size_t* capacity);
  void release(void* p, size_t capacity);
  void trim();  // returns cached blocks to HIP (device must be idle)
  int64_t bytes_in_use() const { return in_use_; }
  int64_t peak_bytes_in_use() const { return peak_; }
  int64_t bytes_reserved() const { return reserved_; }
  int64_t num_allocs() const { return num_allocs_; }
  int64_t largest_alloc() const { return largest_; }

 private:
  int ordinal_;
  std::mutex mu_;
  std::multimap<size_t, void*> free_;
  std::atomic<int64_t> in_use_{0}, peak_{0}, reserved_{0}, num_allocs_{0}, largest_{0};
};

class Device {
 public:
  explicit Device(int ordinal);
  ~Device();
  int ordinal() const { return ordinal_; }
  hipStream_t stream() const { return stream_; }
  Allocator& allocator() { return alloc_; }
  MemRef allocate(size_t bytes);
  void make_current() const;
  std::mutex& exec_mutex() { return exec_mu_; }
  const std::string& arch() const { return arch_; }
  const std::string& name() const { return name_; }
  int64_t total_memory() const { return total_mem_; }
  int compute_units() const { return cus_; }
  // While set (graph capture), every block allocate() hands out is also
  // appended here, so the graph that uses it keeps it for its lifetime.
  void set_capture_pins(std::vector<MemRef>* pins) { capture_pins_ = pins; }
  // Completion events (timing disabled) are reused: an execution records
  // one, and it returns here when the last Event holding it is destroyed.
  hipEvent_t take_event();
  void give_event(hipEvent_t e);
  // A second stream (default priority) for work that runs beside the main
  // stream inside one step, and the two events that fork it from and join it
  // back into the main stream. Created with the device.
  hipStream_t aux_stream() const { return aux_stream_; }
  // Workgroup b of a launch runs on the XCD of workgroup b % 8 (probed when
  // the device is opened).
  bool xcd_round_robin() const { return xcd_round_robin_; }
  hipEvent_t fork_event() const { return fork_ev_; }
  // Arrival counters for library kernels whose last workgroup finishes a
  // launch (one per 128-byte line, kArrivalCounterBytes in all): zeroed when
  // the device is opened; a kernel that counts on a line puts it back to
  // zero before it ends. Launches on the device are ordered on its stream, so
  // they share the lines.
  static constexpr size_t kArrivalCounterBytes = 1 << 20;
  uint32_t* arrival_counters() const { return counters_; }
  hipEvent_t join_event() const { return join_ev_; }
  // A third stream (default priority) with its own fork / join events, for a
  // step that keeps work on the second stream while forking more, and one
  // an event a step may record on a side stream for the main stream to
  // wait on.
  hipStream_t aux2_stream() const { return aux2_stream_; }
  hipEvent_t fork2_event() const { return fork2_ev_; }
  hipEvent_t join2_event() const { return join2_ev_; }
  hipEvent_t side_event() const { return side_ev_; }

 private:
  std::vector<MemRef>* capture_pins_ = nullptr;
  std::mutex ev_mu_;
  std::vector<hipEvent_t> ev_free_;
  int ordinal_;
  hipStream_t stream_ = nullptr;
  hipStream_t aux_stream_ = nullptr;
  hipEvent_t fork_ev_ = nullptr, join_ev_ = nullptr;
  hipStream_t aux2_stream_ = nullptr;
  hipEvent_t fork2_ev_ = nullptr, join2_ev_ = nullptr, side_ev_ = nullptr;
  bool xcd_round_robin_ = false;
  uint32_t* counters_ = nullptr;
  Allocator alloc_;
  std::mutex exec_mu_;
  std::string arch_, name_;
  int64_t total_mem_ = 0;
  int cus_ = 0;
};

// Readiness of device work: pending until a recorded hipEvent completes.
class Event : public std::enable_shared_from_this<Event> {
 public:
  static std::shared_ptr<Event> ready();
  static std::shared_ptr<Event> failed(Code code, const std::string& msg);
  // Marks the stream's current tail. The hipEvent itself is recorded only
  // when readiness is first asked for (see Event::record).
  static std::shared_ptr<Event> record(Device* dev);
  // Resolved by the host later (an async host-to-device transfer that has
  // not received all its data): not ready, and await() blocks, until
  // resolve(then) (it then follows `then`) or resolve_failed().
  static std::shared_ptr<Event> pending();
  void resolve(std::shared_ptr<Event> then);
  void resolve_failed(Code code, const std::string& msg);
  // Blocks until a pending event is resolved (device work it then follows
  // is not waited for; stream order covers it). Throws the failure of an
  // event resolved as failed.
  void wait_resolved();
  ~Event();
  bool is_ready();
  void await();  // blocks until done
  Code error_code() const { return code_; }
  const std::string& error_message() const { return msg_; }
  // Calls fn once the event is done (immediately if it already is).
  void on_ready(std::function<void()> fn);

 private:
  Event() = default;
  // Records the hipEvent of a lazy event (caller holds mu_); false, with the
  // error stored, if recording failed.
  bool materialize_locked();
  std::mutex mu_;
  std::condition_variable cv_;
  bool pending_ = false;          // host-resolved and not yet resolved
  std::shared_ptr<Event> then_;   // what a resolved pending event follows
  hipEvent_t ev_ = nullptr;
  Device* dev_ = nullptr;
  bool lazy_ = false;
  bool done_ = false;
  Code code_ = Code::kOk;
  std::string msg_;
};

struct Buffer {
  Device* dev = nullptr;
  TensorType type;
  MemRef mem;
  std::shared_ptr<Event> ready;
  std::atomic<bool> deleted{false};
};
using BufferRef = std::shared_ptr<Buffer>;

BufferRef buffer_from_host(Device* dev, const TensorType& t, const void* data, const int64_t* byte_strides);

// A program text parsed, rewritten and planned, shared by the compiles of
// the same text under the same PJRTX_* environment (compile_cache.cc).
struct CompiledProgram {
  Program prog;
  Plan plan;
};
std::shared_ptr<const CompiledProgram> compile_program_cached(const std::string& text);
void compile_cache_stats(int64_t* hits, int64_t* misses, int64_t* entries);
void compile_cache_usage(int64_t* bytes, int64_t* evictions);
// The cache key of a program text under the current PJRTX_* environment.
std::string compile_fingerprint(const std::string& text);

// Device residency budget (the reference's executable residency cache:
// src/runtime/executable_cache.zig:85-300, client_residency.zig:58-92):
// every loaded executable's device bytes (code, resident constants, kernel
// scratch) count against a per-device cap (PJRTX_MAX_RESIDENT_BYTES, or
// set_max_resident_bytes; 0 = none). Loading past the cap evicts idle
// executables, the largest first, then the least recently used; an
// executable is busy while it executes.
struct ResidencyStats {
  int64_t resident_bytes = 0, peak_resident_bytes = 0, entries = 0, evictions = 0, evicted_bytes = 0,
          max_resident_bytes = 0;
};
ResidencyStats residency_stats(int ordinal);
void set_max_resident_bytes(int ordinal, int64_t bytes);

// PJRT's asynchronous host-to-device transfer (the reference's async H2D
// manager, src/plugin/async_h2d.zig:196-437): device buffers of fixed
// shapes filled by the host in chunks of any size and order. A chunk is
// copied on the device stream (large ones through the pinned staging ring),
// so executions queued later read it; a buffer becomes ready once its chunk
// flagged `last` has been copied. Until then its readiness event is pending
// (await blocks, an execution taking it waits for it).
class AsyncTransfer {
 public:
  AsyncTransfer(Device* dev, const std::vector<TensorType>& types);
  size_t count() const { return bufs_.size(); }
  size_t bytes(size_t i) const;
  BufferRef buffer(size_t i) const;
  Device* device() const { return dev_; }
  // Copies `size` bytes to [offset, offset + size) of buffer i. Returns the
  // event after which the host may reuse `data`.
  std::shared_ptr<Event> write(size_t i, int64_t offset, const void* data, int64_t size, bool last);
  void fail(size_t i, Code code, const std::string& msg);
  // Buffers still waiting for their last chunk become errors, so that
  // nothing waits on them for ever.
  ~AsyncTransfer();

 private:
  Device* dev_;
  std::mutex mu_;
  std::vector<BufferRef> bufs_;
  // The buffers' device memory, owned here too until each buffer's last
  // chunk: a buffer deleted by its holder mid-transfer keeps its block
  // while a copy into it may still be queued.
  std::vector<MemRef> mems_;
  std::vector<std::shared_ptr<Event>> pending_;  // each buffer's readiness until resolved
  std::vector<bool> finished_;
};

// Large host-to-device copies through a pinned staging ring on a copy
// stream (transfer.cc); returns when the data is on the device.
bool staged_upload_wanted(size_t bytes);
void staged_upload(Device* dev, void* dst, const void* src, size_t bytes);
// Large device-to-host copies through the same ring; returns when the data
// is in `dst`.
bool staged_download_wanted(size_t bytes);
void staged_download(Device* dev, void* dst, const void* src, size_t bytes);
void buffer_to_host(const Buffer& b, void* dst, size_t dst_size);

// hiprtc compile of generated kernel source for the device arch, cached in
// memory and on disk (PJRTX_KERNEL_CACHE_DIR, default ~/.cache/pjrtx_amd).
std::vector<char> compile_kernels(const std::string& source, const std::string& arch);
// The full translation unit hiprtc sees: device helper header + body.
std::string kernel_translation_unit(const std::string& body);

struct ExecStats {
  int64_t executions = 0;
  int64_t kernel_launches = 0;
  int64_t library_calls = 0;
  int64_t released_values = 0;
  int64_t graph_captures = 0;
  int64_t graph_replays = 0;
};

class Executable {
 public:
  Executable(Program prog, Plan plan, std::string fingerprint, std::string name);
  ~Executable();
  // Loads code and resident constants on `dev` (once).
  void load(Device* dev);
  // Runs the plan; inputs must be on `dev`. Returns one buffer per result.
  // `donate[i]` true hands argument i's memory to this execution: a step may
  // write it in place and a result may keep it (the caller must treat the
  // argument as deleted). A parameter the plan writes in place but whose
  // argument is not donated is copied first.
  std::vector<BufferRef> execute(Device* dev, const std::vector<BufferRef>& args,
                                 std::shared_ptr<Event>* done, const std::vector<bool>* donate = nullptr);
  // The same plan on caller-owned device memory with no allocation: args[i]
  // and outs[i] are device addresses of the parameter / result sizes; every
  // intermediate, copy of a parameter the plan writes, and kernel scratch
  // block comes from the device's fixed no-allocation block (kernels/
  // noalloc.h), whose contents the previous call left behind. Work is queued
  // on the device stream (no graph capture, no completion event). The
  // executable must already be loaded on `dev`. Returns the arena bytes used.
  size_t execute_noalloc(Device* dev, const void* const* args, size_t num_args, void* const* outs,
                         size_t num_outs);
  // Times each launch unit (a step; a split reduction counts as two units,
  // main pass then combine pass) by replaying it `iters` times between two
  // hipEvents on the device stream (inputs from `args`). Returns ms per unit
  // in the order of unit_names().
  std::vector<double> time_steps(Device* dev, const std::vector<BufferRef>& args, int iters);
  // Kernel name of each launch unit ("lib:<kind>" for library steps).
  std::vector<std::string> unit_names() const;
  // Runs the plan on device memory: `args` bound to the parameters, one
  // block per result (a result may be an argument's block). Used for the
  // regions of a while loop; the caller holds the device's execute lock.
  std::vector<MemRef> run_values(Device* dev, const std::vector<MemRef>& args);
  // Iteration count of the while step `si` when constants fix it, else -1.
  int64_t while_trips(size_t si) const;

  const Program& program() const { return prog_; }
  const Plan& plan() const { return plan_; }
  const std::string& fingerprint() const { return fingerprint_; }
  const std::string& name() const { return name_; }
  size_t code_size() const { return code_.size(); }
  ExecStats stats() const { return stats_; }
  // Drops this executable's device state on `ordinal` (code, resident
  // constants, kernel scratch, captured graphs); the next execution there
  // loads it again. Called by the residency budget on an idle executable.
  void evict(int ordinal);

 private:
  struct Loaded {
    Device* dev = nullptr;
    hipModule_t module = nullptr;
    std::vector<hipFunction_t> funcs;          // per step (null for non-kernel)
    std::vector<hipFunction_t> combine_funcs;  // split reductions: second pass
    std::map<int, MemRef> constants;           // value id -> resident buffer
    std::vector<MemRef> scratch;               // per step partials
  };
  // A while loop's cond and body compiled as programs of their own
  // (parameters: the loop state, then the values the regions capture), and
  // its iteration count when constants fix it (-1 otherwise).
  struct WhileLoop {
    std::unique_ptr<Executable> cond, body;
    int64_t trips = -1;
  };
  void run_while(Loaded* L, size_t si, std::vector<MemRef>& vals);

  Program prog_;
  Plan plan_;
  std::map<size_t, std::unique_ptr<WhileLoop>> loops_;
  std::string fingerprint_, name_;
  std::vector<char> code_;
  std::mutex mu_;
  std::map<int, std::unique_ptr<Loaded>> loaded_;
  ExecStats stats_;

  // A captured hipGraph of the whole plan for one set of argument
  // addresses. Small arguments are staged into pinned blocks before each
  // replay; results the graph produces are copied out to fresh buffers.
  struct GraphEntry {
    std::vector<const void*> key;  // per parameter: device address, or null when staged
    hipGraphExec_t exec = nullptr;
    std::vector<MemRef> pins;      // every block the graph reads or writes
    std::vector<MemRef> staging;   // per parameter: staging block (staged parameters)
    std::vector<int> result_param; // per result: parameter whose memory it is, or -1
    std::vector<MemRef> result_mem;
    uint64_t last_use = 0;
    ~GraphEntry();
  };
  struct GraphState {
    std::vector<std::unique_ptr<GraphEntry>> entries;
    std::vector<std::vector<const void*>> seen;  // keys run once eagerly
    bool disabled = false;
    uint64_t clock = 0;
  };
  std::map<int, GraphState> graphs_;  // by device ordinal

  // `may_evict`: the caller holds the device's execute lock, so idle
  // executables may be evicted to keep within the residency budget.
  Loaded* loaded_for(Device* dev, bool may_evict = false);
  GraphState& graph_state(int ordinal);
  bool graph_candidate(const std::vector<BufferRef>& args, const std::vector<bool>* donate) const;
  std::vector<const void*> graph_key(const std::vector<BufferRef>& args) const;
  GraphEntry* capture_graph(Device* dev, Loaded* L, const std::vector<BufferRef>& args,
                            std::vector<const void*> key);
  std::vector<BufferRef> replay_graph(Device* dev, GraphEntry* g, const std::vector<BufferRef>& args,
                                      std::shared_ptr<Event>* done);
  // phase: -1 runs the whole step; 0 only the main kernel of a split
  // reduction, 1 only its combine kernel (outputs must already exist).
  void run_step(Loaded* L, size_t si, std::vector<MemRef>& vals, int phase = -1);
};

// Library steps (dot_general, gather, scatter, dynamic slices, ...).
void run_library_step(Device* dev, const Program& prog, const Step& step,
                      std::vector<MemRef>& vals);

}  // namespace pjrtx
