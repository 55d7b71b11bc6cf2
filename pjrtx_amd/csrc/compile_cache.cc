// Compile cache (the reference's executable cache: src/runtime/
// executable_cache.zig, keyed by program fingerprint). A program text that
// was compiled before, under the same PJRTX_* environment (the switches
// that change plans), reuses its parsed, rewritten and planned form; each
// compile still builds its own Executable (own statistics, graphs and
// loaded module), so sharing is invisible to callers. Kernel code objects
// are cached separately by source hash (in process and on disk). Entries
// are evicted least recently used.
#include <unistd.h>

#include <cstring>

#include <list>
#include <mutex>
#include <unordered_map>

#include "planner.h"
#include "runtime.h"

extern char** environ;

namespace pjrtx {
namespace {

constexpr size_t kCapacity = 32;

struct Cache {
  std::mutex mu;
  std::list<std::string> lru;  // most recent first
  std::unordered_map<std::string, std::pair<std::shared_ptr<const CompiledProgram>, std::list<std::string>::iterator>>
      map;
  int64_t hits = 0, misses = 0;
};

Cache& cache() {
  static Cache* c = new Cache();
  return *c;
}

std::string env_key() {
  std::string k;
  for (char** e = environ; e && *e; ++e)
    if (std::strncmp(*e, "PJRTX_", 6) == 0) k += std::string(*e) + '\n';
  return k;
}

}  // namespace

std::shared_ptr<const CompiledProgram> compile_program_cached(const std::string& text) {
  const std::string key = env_key() + '\0' + text;
  Cache& c = cache();
  {
    std::lock_guard<std::mutex> lk(c.mu);
    auto it = c.map.find(key);
    if (it != c.map.end()) {
      c.lru.splice(c.lru.begin(), c.lru, it->second.second);
      c.hits++;
      return it->second.first;
    }
  }
  auto cp = std::make_shared<CompiledProgram>();
  cp->prog = parse_stablehlo(text);
  rewrite_program(&cp->prog);
  cp->plan = make_plan(cp->prog);
  std::lock_guard<std::mutex> lk(c.mu);
  c.misses++;
  if (!c.map.count(key)) {
    c.lru.push_front(key);
    c.map[key] = {cp, c.lru.begin()};
    while (c.map.size() > kCapacity) {
      c.map.erase(c.lru.back());
      c.lru.pop_back();
    }
  }
  return cp;
}

void compile_cache_stats(int64_t* hits, int64_t* misses, int64_t* entries) {
  Cache& c = cache();
  std::lock_guard<std::mutex> lk(c.mu);
  if (hits) *hits = c.hits;
  if (misses) *misses = c.misses;
  if (entries) *entries = static_cast<int64_t>(c.map.size());
}

}  // namespace pjrtx
