// Compile cache (the reference's executable cache: src/runtime/
// executable_cache.zig:85-300, keyed by the fingerprint of
// executable_fingerprint.zig:9-24). A program text that was compiled before,
// under the same PJRTX_* environment (the switches that change plans),
// reuses its parsed, rewritten and planned form; each compile still builds
// its own Executable (own statistics, graphs and loaded module), so sharing
// is invisible to callers. The key is a 128-bit fingerprint of environment
// and text ("pjrtx-" + two FNV-1a hashes), so a cached entry does not hold
// its text twice. Entries are evicted least recently used once there are
// more than 32 or their host bytes (text plus constant literals) pass
// PJRTX_COMPILE_CACHE_BYTES (default 256 MiB). Kernel code objects are
// cached separately by source hash (in process and on disk).
#include <unistd.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>

#include <list>
#include <mutex>
#include <unordered_map>

#include "custom_call.h"
#include "planner.h"
#include "runtime.h"

extern char** environ;

namespace pjrtx {
namespace {

constexpr size_t kCapacity = 32;

struct Entry {
  std::shared_ptr<const CompiledProgram> cp;
  std::list<std::string>::iterator pos;
  int64_t bytes = 0;
};

struct Cache {
  std::mutex mu;
  std::list<std::string> lru;  // most recent first
  std::unordered_map<std::string, Entry> map;
  int64_t hits = 0, misses = 0, bytes = 0, evictions = 0;
};

int64_t byte_cap() {
  const char* v = std::getenv("PJRTX_COMPILE_CACHE_BYTES");
  return v && *v ? std::atoll(v) : (int64_t(256) << 20);
}

uint64_t fnv1a64(const std::string& s, uint64_t h) {
  for (unsigned char c : s) {
    h ^= c;
    h *= 1099511628211ull;
  }
  return h;
}

std::string fingerprint(const std::string& src) {
  char buf[48];
  std::snprintf(buf, sizeof buf, "pjrtx-%016llx%016llx",
                static_cast<unsigned long long>(fnv1a64(src, 1469598103934665603ull)),
                static_cast<unsigned long long>(fnv1a64(src, 0x9e3779b97f4a7c15ull)));
  return buf;
}

int64_t host_bytes(const std::string& text, const Program& prog) {
  int64_t b = static_cast<int64_t>(text.size());
  for (const Op& op : prog.ops) b += static_cast<int64_t>(op.literal.size());
  return b;
}

Cache& cache() {
  static Cache* c = new Cache();
  return *c;
}

std::string env_key() {
  std::string k;
  for (char** e = environ; e && *e; ++e)
    if (std::strncmp(*e, "PJRTX_", 6) == 0) k += std::string(*e) + '\n';
  // Registered custom-call targets change how a program lowers.
  k += "custom_call_registry " + std::to_string(custom_call_registry_version()) + '\n';
  return k;
}

}  // namespace

std::shared_ptr<const CompiledProgram> compile_program_cached(const std::string& text) {
  const std::string key = fingerprint(env_key() + '\0' + text);
  Cache& c = cache();
  {
    std::lock_guard<std::mutex> lk(c.mu);
    auto it = c.map.find(key);
    if (it != c.map.end()) {
      c.lru.splice(c.lru.begin(), c.lru, it->second.pos);
      c.hits++;
      return it->second.cp;
    }
  }
  auto cp = std::make_shared<CompiledProgram>();
  cp->prog = parse_stablehlo(text);
  rewrite_program(&cp->prog);
  cp->plan = make_plan(cp->prog);
  const int64_t bytes = host_bytes(text, cp->prog);
  const int64_t cap = byte_cap();
  std::lock_guard<std::mutex> lk(c.mu);
  c.misses++;
  if (!c.map.count(key) && bytes <= cap) {
    c.lru.push_front(key);
    c.map[key] = Entry{cp, c.lru.begin(), bytes};
    c.bytes += bytes;
    while (c.map.size() > kCapacity || c.bytes > cap) {
      auto victim = c.map.find(c.lru.back());
      c.bytes -= victim->second.bytes;
      c.evictions++;
      c.map.erase(victim);
      c.lru.pop_back();
    }
  }
  return cp;
}

std::string compile_fingerprint(const std::string& text) { return fingerprint(env_key() + '\0' + text); }

void compile_cache_stats(int64_t* hits, int64_t* misses, int64_t* entries) {
  Cache& c = cache();
  std::lock_guard<std::mutex> lk(c.mu);
  if (hits) *hits = c.hits;
  if (misses) *misses = c.misses;
  if (entries) *entries = static_cast<int64_t>(c.map.size());
}

void compile_cache_usage(int64_t* bytes, int64_t* evictions) {
  Cache& c = cache();
  std::lock_guard<std::mutex> lk(c.mu);
  if (bytes) *bytes = c.bytes;
  if (evictions) *evictions = c.evictions;
}

}  // namespace pjrtx
