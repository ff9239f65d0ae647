// rxmet_prof.cpp — event timing of instrumented kernel launches (rxmet_prof.h).
#include "rxmet_prof.h"

#include <hip/hip_runtime.h>

#include <cstring>
#include <map>
#include <mutex>
#include <string>
#include <utility>
#include <vector>

#include "rxmet_common.h"

namespace rxmet {
namespace prof {
namespace {

struct Entry {
  double ms = 0.0;
  int64_t launches = 0;
  std::vector<std::pair<hipEvent_t, hipEvent_t>> pending;
};

std::mutex g_mu;
bool g_on = false;
std::map<std::string, Entry> g_entries;
std::vector<hipEvent_t> g_pool;
constexpr size_t kPrewarm = 4096;  // events kept ready while timing is on
std::vector<std::string> g_filter;  // names timed; empty: all

hipEvent_t take_event() {
  if (!g_pool.empty()) {
    hipEvent_t e = g_pool.back();
    g_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

void resolve(Entry &en) {
  for (auto &pr : en.pending) {
    float ms = 0.0f;
    if (hipEventSynchronize(pr.second) == hipSuccess &&
        hipEventElapsedTime(&ms, pr.first, pr.second) == hipSuccess) {
      en.ms += ms;
      en.launches += 1;
    }
    g_pool.push_back(pr.first);
    g_pool.push_back(pr.second);
  }
  en.pending.clear();
}

}  // namespace

bool enabled() { return g_on; }

Scope::Scope(const char *name, hipStream_t stream) : name_(name), stream_(stream) {
  if (!g_on) return;
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_filter.empty()) {
    bool hit = false;
    for (const std::string &f : g_filter) hit = hit || f == name_;
    if (!hit) return;
  }
  start_ = take_event();
  if (start_ && hipEventRecord(start_, stream_) != hipSuccess) {
    g_pool.push_back(start_);
    start_ = nullptr;
  }
}

Scope::~Scope() {
  if (!start_) return;
  std::lock_guard<std::mutex> lk(g_mu);
  hipEvent_t stop = take_event();
  if (!stop || hipEventRecord(stop, stream_) != hipSuccess) {
    g_pool.push_back(start_);
    if (stop) g_pool.push_back(stop);
    return;
  }
  g_entries[name_].pending.emplace_back(start_, stop);
}

}  // namespace prof
}  // namespace rxmet

using namespace rxmet::prof;

extern "C" {

int rxmet_prof_enable(int32_t on) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_on = on != 0;
  // events are created up front, so that timed launches only take them from the pool
  // (creating one per launch costs host time inside the timed region)
  for (size_t i = g_pool.size(); g_on && i < kPrewarm; ++i) {
    hipEvent_t e = nullptr;
    if (hipEventCreate(&e) != hipSuccess) break;
    g_pool.push_back(e);
  }
  return 0;
}

int rxmet_prof_filter(const char *names) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_filter.clear();
  if (names == nullptr) return 0;
  std::string cur;
  for (const char *c = names;; ++c) {
    if (*c == ',' || *c == '\0') {
      if (!cur.empty()) g_filter.push_back(cur);
      cur.clear();
      if (*c == '\0') break;
    } else {
      cur += *c;
    }
  }
  return 0;
}

int rxmet_prof_reset(void) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto &kv : g_entries) {
    for (auto &pr : kv.second.pending) {
      (void)hipEventSynchronize(pr.second);
      g_pool.push_back(pr.first);
      g_pool.push_back(pr.second);
    }
  }
  g_entries.clear();
  return 0;
}

int rxmet_prof_query(const char *name, double *total_ms, int64_t *launches) {
  std::lock_guard<std::mutex> lk(g_mu);
  double ms = 0.0;
  int64_t n = 0;
  auto it = name ? g_entries.find(name) : g_entries.end();
  if (it != g_entries.end()) {
    resolve(it->second);
    ms = it->second.ms;
    n = it->second.launches;
  }
  if (total_ms) *total_ms = ms;
  if (launches) *launches = n;
  return 0;
}

int64_t rxmet_prof_names(char *buf, int64_t len) {
  std::lock_guard<std::mutex> lk(g_mu);
  std::string all;
  for (auto &kv : g_entries) {
    if (!all.empty()) all += ",";
    all += kv.first;
  }
  if (buf && len > 0) {
    const size_t n = std::min(static_cast<size_t>(len - 1), all.size());
    std::memcpy(buf, all.data(), n);
    buf[n] = '\0';
  }
  return static_cast<int64_t>(all.size());
}

}  // extern "C"
