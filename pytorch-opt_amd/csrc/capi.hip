// C-ABI plumbing: last-error strings, version, and HIP-event timing of
// individual kernel classes (used by the benchmark to report the average
// launch duration of the dominant kernel).
#include <mutex>
#include <string>
#include <unordered_map>
#include <vector>

#include "pto_common.h"

namespace pto {

static thread_local std::string g_last_error;

void set_error(const std::string& msg) { g_last_error = msg; }

namespace {

struct EventPair {
  hipEvent_t start, stop;
};

struct ProfState {
  std::mutex mu;
  bool enabled = false;
  std::vector<hipEvent_t> pool;  // recycled events
  std::unordered_map<std::string, std::vector<EventPair>> pending;
  std::unordered_map<std::string, std::pair<double, int64_t>> totals;  // ms, launches
};

ProfState& prof() {
  static ProfState* s = new ProfState();  // never destroyed: safe at exit
  return *s;
}

hipEvent_t take_event(ProfState& p) {
  if (!p.pool.empty()) {
    hipEvent_t e = p.pool.back();
    p.pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

struct Token {
  std::string name;
  hipEvent_t start;
};

// Resolve every recorded pair into the totals (blocks on the events).
int drain(ProfState& p) {
  int rc = 0;
  for (auto& kv : p.pending) {
    auto& tot = p.totals[kv.first];
    for (auto& ev : kv.second) {
      float ms = 0.f;
      if (hipEventSynchronize(ev.stop) != hipSuccess || hipEventElapsedTime(&ms, ev.start, ev.stop) != hipSuccess)
        rc = -1;
      tot.first += ms;
      tot.second += 1;
      p.pool.push_back(ev.start);
      p.pool.push_back(ev.stop);
    }
    kv.second.clear();
  }
  return rc;
}

}  // namespace

static thread_local int g_prof_suspended = 0;

bool prof_enabled() { return g_prof_suspended == 0 && prof().enabled; }

void prof_suspend(int delta) { g_prof_suspended += delta; }

void prof_begin(const char* name, hipStream_t stream, void** token) {
  ProfState& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  hipEvent_t e = take_event(p);
  if (e == nullptr) return;
  if (hipEventRecord(e, stream) != hipSuccess) {
    p.pool.push_back(e);
    return;
  }
  *token = new Token{name, e};
}

void prof_end(void* token, hipStream_t stream) {
  Token* t = static_cast<Token*>(token);
  ProfState& p = prof();
  std::lock_guard<std::mutex> lk(p.mu);
  hipEvent_t e = take_event(p);
  if (e != nullptr && hipEventRecord(e, stream) == hipSuccess) {
    p.pending[t->name].push_back(EventPair{t->start, e});
  } else {
    p.pool.push_back(t->start);
    if (e) p.pool.push_back(e);
  }
  delete t;
}

}  // namespace pto

extern "C" {

const char* pto_last_error(void) { return pto::g_last_error.c_str(); }

int pto_version(void) { return 10000; }  // 1.0.0

int pto_runtime_version(void) {
  int v = 0;
  if (hipRuntimeGetVersion(&v) != hipSuccess) return -1;
  return v;
}

int pto_prof_enable(int on) {
  pto::ProfState& p = pto::prof();
  std::lock_guard<std::mutex> lk(p.mu);
  p.enabled = on != 0;
  return 0;
}

int pto_prof_reset(void) {
  pto::ProfState& p = pto::prof();
  std::lock_guard<std::mutex> lk(p.mu);
  int rc = pto::drain(p);
  p.totals.clear();
  return rc;
}

int pto_prof_query(const char* name, double* total_ms, int64_t* launches) {
  pto::ProfState& p = pto::prof();
  std::lock_guard<std::mutex> lk(p.mu);
  PTO_REQUIRE(name != nullptr && total_ms != nullptr && launches != nullptr, "pto_prof_query: null argument");
  if (pto::drain(p) != 0) {
    pto::set_error("pto_prof_query: event timing failed");
    return -1;
  }
  auto it = p.totals.find(name);
  *total_ms = it == p.totals.end() ? 0.0 : it->second.first;
  *launches = it == p.totals.end() ? 0 : it->second.second;
  return 0;
}

}  // extern "C"
