// pjrtx_hip_* C ABI (declared in include/pjrtx_hip.h).
#include <chrono>
#include <cstring>
#include <map>
#include <mutex>

#include "../../include/pjrt_c_api.h"
#include "../../include/pjrtx_hip.h"
#include "pjrt_handles.h"
#include "runtime.h"
#include "kernels/library.h"
#include "kernels/noalloc.h"

using namespace pjrtx;

namespace {
thread_local std::string g_last_error;

template <typename Fn>
int guarded(Fn&& fn) {
  try {
    fn();
    return 0;
  } catch (const Error& e) {
    g_last_error = e.what();
    return static_cast<int>(e.code);
  } catch (const std::exception& e) {
    g_last_error = e.what();
    return static_cast<int>(Code::kInternal);
  }
}

std::mutex g_mu;
std::map<int, std::unique_ptr<Device>> g_abi_devices;
std::map<void*, MemRef> g_abi_allocs;

Device* abi_device(int ordinal) {
  std::lock_guard<std::mutex> lk(g_mu);
  auto it = g_abi_devices.find(ordinal);
  if (it != g_abi_devices.end()) return it->second.get();
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || ordinal < 0 || ordinal >= n) {
    (void)hipGetLastError();
    fail(Code::kFailedPrecondition, strformat("no HIP device %d", ordinal));
  }
  auto d = std::make_unique<Device>(ordinal);
  Device* raw = d.get();
  g_abi_devices[ordinal] = std::move(d);
  return raw;
}

void copy_out(const std::string& s, char* out, size_t cap, size_t* needed) {
  if (needed) *needed = s.size() + 1;
  if (out && cap) {
    const size_t n = std::min(cap - 1, s.size());
    std::memcpy(out, s.data(), n);
    out[n] = '\0';
  }
}
}  // namespace

extern "C" const PJRT_Api* GetPjrtApi(void);

extern "C" {

const char* pjrtx_hip_last_error(void) { return g_last_error.c_str(); }

int pjrtx_hip_device_count(int* count) {
  return guarded([&] {
    int n = 0;
    if (hipGetDeviceCount(&n) != hipSuccess) {
      (void)hipGetLastError();
      n = 0;
    }
    *count = n;
  });
}

int pjrtx_hip_malloc(int device, size_t bytes, void** ptr) {
  return guarded([&] {
    MemRef m = abi_device(device)->allocate(bytes);
    std::lock_guard<std::mutex> lk(g_mu);
    *ptr = m->ptr;
    if (m->ptr) g_abi_allocs[m->ptr] = m;
  });
}

int pjrtx_hip_free(int device, void* ptr) {
  return guarded([&] {
    (void)device;
    std::lock_guard<std::mutex> lk(g_mu);
    auto it = g_abi_allocs.find(ptr);
    PJRTX_CHECK(it != g_abi_allocs.end(), Code::kInvalidArgument, "pjrtx_hip_free: unknown pointer");
    g_abi_allocs.erase(it);
  });
}

int pjrtx_hip_copy_h2d(int device, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    Device* d = abi_device(device);
    d->make_current();
    hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, d->stream()), "hipMemcpyAsync(H2D)");
    hip_check(hipStreamSynchronize(d->stream()), "hipStreamSynchronize");
  });
}

int pjrtx_hip_copy_d2h(int device, void* dst, const void* src, size_t bytes) {
  return guarded([&] {
    Device* d = abi_device(device);
    d->make_current();
    hip_check(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, d->stream()), "hipMemcpyAsync(D2H)");
    hip_check(hipStreamSynchronize(d->stream()), "hipStreamSynchronize");
  });
}

int pjrtx_hip_synchronize(int device) {
  return guarded([&] {
    Device* d = abi_device(device);
    d->make_current();
    // Every stream of the device: PJRT clients and this ABI queue on streams
    // of their own.
    hip_check(hipDeviceSynchronize(), "hipDeviceSynchronize");
  });
}

int pjrtx_compile_cache_stats(int64_t* hits, int64_t* misses, int64_t* entries) {
  return guarded([&] { compile_cache_stats(hits, misses, entries); });
}

int pjrtx_mfma_peak_tflops(int device, int shape, double* tflops) {
  return guarded([&] {
    PJRTX_CHECK(tflops != nullptr, Code::kInvalidArgument, "mfma_peak_tflops: null output");
    Device* d = abi_device(device);
    d->make_current();
    std::lock_guard<std::mutex> lk(d->exec_mutex());
    *tflops = measure_mfma_peak_tflops(d->stream(), shape, d->compute_units());
  });
}

int pjrtx_compile_cache_usage(int64_t* bytes, int64_t* evictions) {
  return guarded([&] { compile_cache_usage(bytes, evictions); });
}

int pjrtx_compile_fingerprint(const char* text, size_t len, char* out, size_t cap, size_t* needed) {
  return guarded([&] { copy_out(compile_fingerprint(std::string(text, len)), out, cap, needed); });
}

int pjrtx_set_max_resident_bytes(int device, int64_t bytes) {
  return guarded([&] {
    PJRTX_CHECK(bytes >= 0, Code::kInvalidArgument, "set_max_resident_bytes: negative cap");
    set_max_resident_bytes(abi_device(device)->ordinal(), bytes);
  });
}

int pjrtx_residency_stats(int device, int64_t out[6]) {
  return guarded([&] {
    PJRTX_CHECK(out != nullptr, Code::kInvalidArgument, "residency_stats: null output");
    const ResidencyStats st = residency_stats(abi_device(device)->ordinal());
    out[0] = st.resident_bytes;
    out[1] = st.peak_resident_bytes;
    out[2] = st.entries;
    out[3] = st.evictions;
    out[4] = st.evicted_bytes;
    out[5] = st.max_resident_bytes;
  });
}

int pjrtx_plan_json(const char* text, size_t len, char* out, size_t cap, size_t* needed) {
  return guarded([&] {
    Program prog = parse_stablehlo(std::string(text, len));
    rewrite_program(&prog);
    Plan plan = make_plan(prog);
    copy_out(plan.describe(prog), out, cap, needed);
  });
}

int pjrtx_compile_check(const char* text, size_t len, const char* arch, size_t* code_size) {
  return guarded([&] {
    Program prog = parse_stablehlo(std::string(text, len));
    rewrite_program(&prog);
    Plan plan = make_plan(prog);
    size_t n = 0;
    if (plan.num_fusion_kernels > 0) n = compile_kernels(plan.kernel_source, arch ? arch : "gfx950").size();
    if (code_size) *code_size = n;
  });
}

int pjrtx_kernel_source(const char* text, size_t len, char* out, size_t cap, size_t* needed) {
  return guarded([&] {
    Program prog = parse_stablehlo(std::string(text, len));
    rewrite_program(&prog);
    Plan plan = make_plan(prog);
    copy_out(kernel_translation_unit(plan.kernel_source), out, cap, needed);
  });
}

int pjrtx_executable_time_steps(PJRT_LoadedExecutable* exe, PJRT_Buffer* const* args, size_t num_args, int iters,
                                double* ms, size_t cap, size_t* steps) {
  return guarded([&] {
    PJRTX_CHECK(exe && iters > 0, Code::kInvalidArgument, "time_steps: bad arguments");
    std::vector<BufferRef> in;
    for (size_t i = 0; i < num_args; ++i) in.push_back(args[i]->buf);
    Device* dev = in.empty() ? exe->devices.at(0)->dev : in[0]->dev;
    std::vector<double> t = exe->exe->time_steps(dev, in, iters);
    if (steps) *steps = t.size();
    for (size_t i = 0; i < t.size() && i < cap; ++i) ms[i] = t[i];
  });
}

int pjrtx_executable_run(PJRT_LoadedExecutable* exe, PJRT_Buffer* const* args, size_t num_args, int iters,
                         double* ms_total) {
  return guarded([&] {
    PJRTX_CHECK(exe && iters > 0 && ms_total, Code::kInvalidArgument, "run: bad arguments");
    PJRTX_CHECK(!exe->deleted, Code::kFailedPrecondition, "run: executable was deleted");
    std::vector<BufferRef> in;
    for (size_t i = 0; i < num_args; ++i) {
      PJRTX_CHECK(args[i] && !args[i]->buf->deleted, Code::kInvalidArgument, "run: argument is null or deleted");
      in.push_back(args[i]->buf);
    }
    Device* dev = in.empty() ? exe->devices.at(0)->dev : in[0]->dev;
    dev->make_current();
    hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize");
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < iters; ++i) {
      std::shared_ptr<Event> done;
      std::vector<BufferRef> outs = exe->exe->execute(dev, in, &done, nullptr);
    }
    hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize");
    *ms_total = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  });
}

int pjrtx_executable_run_pjrt(PJRT_LoadedExecutable* exe, PJRT_Buffer* const* args, size_t num_args, int iters,
                              double* ms_total) {
  return guarded([&] {
    PJRTX_CHECK(exe && iters > 0 && ms_total, Code::kInvalidArgument, "run_pjrt: bad arguments");
    PJRTX_CHECK(!exe->deleted, Code::kFailedPrecondition, "run_pjrt: executable was deleted");
    PJRTX_CHECK(args || num_args == 0, Code::kInvalidArgument, "run_pjrt: null argument array");
    const PJRT_Api* api = GetPjrtApi();
    Device* dev = num_args ? args[0]->buf->dev : exe->devices.at(0)->dev;
    const size_t nout = exe->exe->program().results.size();
    std::vector<PJRT_Buffer*> outs(std::max<size_t>(1, nout));
    PJRT_Buffer** out_lists[1] = {outs.data()};
    PJRT_Buffer* const* arg_lists[1] = {args};
    PJRT_Event* events[1] = {nullptr};
    PJRT_ExecuteOptions opts;
    std::memset(&opts, 0, sizeof(opts));
    opts.struct_size = PJRT_ExecuteOptions_STRUCT_SIZE;
    PJRT_LoadedExecutable_Execute_Args a;
    std::memset(&a, 0, sizeof(a));
    a.struct_size = PJRT_LoadedExecutable_Execute_Args_STRUCT_SIZE;
    a.executable = exe;
    a.options = &opts;
    a.argument_lists = arg_lists;
    a.num_devices = 1;
    a.num_args = num_args;
    a.output_lists = out_lists;
    a.device_complete_events = events;
    // A PJRT error from the loop is returned as this call's status.
    auto call = [&](PJRT_Error* e) {
      if (!e) return;
      PJRT_Error_Message_Args m;
      std::memset(&m, 0, sizeof(m));
      m.struct_size = PJRT_Error_Message_Args_STRUCT_SIZE;
      m.error = e;
      api->PJRT_Error_Message(&m);
      const std::string msg(m.message, m.message_size);
      PJRT_Error_Destroy_Args d;
      std::memset(&d, 0, sizeof(d));
      d.struct_size = PJRT_Error_Destroy_Args_STRUCT_SIZE;
      d.error = e;
      api->PJRT_Error_Destroy(&d);
      fail(Code::kInternal, "run_pjrt: " + msg);
    };
    dev->make_current();
    hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize");
    const auto t0 = std::chrono::steady_clock::now();
    for (int i = 0; i < iters; ++i) {
      call(api->PJRT_LoadedExecutable_Execute(&a));
      if (events[0]) {
        PJRT_Event_Destroy_Args ed;
        std::memset(&ed, 0, sizeof(ed));
        ed.struct_size = PJRT_Event_Destroy_Args_STRUCT_SIZE;
        ed.event = events[0];
        call(api->PJRT_Event_Destroy(&ed));
        events[0] = nullptr;
      }
      for (size_t k = 0; k < nout; ++k) {
        PJRT_Buffer_Destroy_Args bd;
        std::memset(&bd, 0, sizeof(bd));
        bd.struct_size = PJRT_Buffer_Destroy_Args_STRUCT_SIZE;
        bd.buffer = outs[k];
        call(api->PJRT_Buffer_Destroy(&bd));
      }
    }
    hip_check(hipStreamSynchronize(dev->stream()), "hipStreamSynchronize");
    *ms_total = std::chrono::duration<double, std::milli>(std::chrono::steady_clock::now() - t0).count();
  });
}

int pjrtx_executable_execute_noalloc(PJRT_LoadedExecutable* exe, int device, const void* const* args,
                                     size_t num_args, void* const* outputs, size_t num_outputs,
                                     size_t* scratch_used) {
  return guarded([&] {
    PJRTX_CHECK(exe && exe->exe, Code::kInvalidArgument, "execute_noalloc: null executable");
    PJRTX_CHECK(!exe->deleted, Code::kFailedPrecondition, "execute_noalloc: executable was deleted");
    PJRTX_CHECK((args || num_args == 0) && (outputs || num_outputs == 0), Code::kInvalidArgument,
                "execute_noalloc: null argument or output array");
    Device* dev = nullptr;
    for (PJRT_Device* d : exe->devices)
      if (d && d->dev && d->dev->ordinal() == device) dev = d->dev;
    PJRTX_CHECK(dev != nullptr, Code::kInvalidArgument,
                strformat("execute_noalloc: the executable is not addressable on device %d", device));
    const size_t used = exe->exe->execute_noalloc(dev, args, num_args, outputs, num_outputs);
    if (scratch_used) *scratch_used = used;
  });
}

size_t pjrtx_noalloc_scratch_bytes(void) { return kNoallocScratchBytes; }

int pjrtx_executable_step_names(PJRT_LoadedExecutable* exe, char* out, size_t cap, size_t* needed) {
  return guarded([&] {
    std::string s;
    for (const std::string& n : exe->exe->unit_names()) s += n + "\n";
    copy_out(s, out, cap, needed);
  });
}

int pjrtx_executable_stats(PJRT_LoadedExecutable* exe, int64_t out[4]) {
  return guarded([&] {
    ExecStats s = exe->exe->stats();
    out[0] = s.executions;
    out[1] = s.kernel_launches;
    out[2] = s.library_calls;
    out[3] = s.released_values;
  });
}

int pjrtx_executable_graph_stats(PJRT_LoadedExecutable* exe, int64_t out[2]) {
  return guarded([&] {
    ExecStats s = exe->exe->stats();
    out[0] = s.graph_captures;
    out[1] = s.graph_replays;
  });
}

}  // extern "C"
