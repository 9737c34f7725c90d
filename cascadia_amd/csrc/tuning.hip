// tuning.hip -- a process-wide cache of the CASCADIA_INT4_* tuning variables,
// so that the per-call host path reads no environment.
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <mutex>

#include "../../include/cascadia_int4.h"
#include "tuning.hpp"

namespace {

constexpr int kMaxKnobs = 32;

struct Knob {
  const char *name;  // a string literal: compared by address first
  bool set;          // the variable was present and numeric
  int value;
  unsigned gen;      // g_gen when it was read
};

std::mutex g_knob_mu;
Knob g_knobs[kMaxKnobs];
int g_n_knobs = 0;
std::atomic<unsigned> g_gen{1};

bool read_env(const char *name, int *out) {
  const char *e = getenv(name);
  if (!e) return false;
  char *end = nullptr;
  const long v = strtol(e, &end, 10);
  if (end == e) return false;
  *out = (int)v;
  return true;
}

}  // namespace

namespace cai4 {

int tuning_env(const char *name, int absent) {
  const unsigned gen = g_gen.load(std::memory_order_acquire);
  std::lock_guard<std::mutex> lk(g_knob_mu);
  Knob *k = nullptr;
  for (int i = 0; i < g_n_knobs; i++)
    if (g_knobs[i].name == name || strcmp(g_knobs[i].name, name) == 0) {
      k = &g_knobs[i];
      break;
    }
  if (!k) {
    if (g_n_knobs == kMaxKnobs) {  // not expected: read it uncached
      int v;
      return read_env(name, &v) ? v : absent;
    }
    k = &g_knobs[g_n_knobs++];
    k->name = name;
    k->gen = 0;
  }
  if (k->gen != gen) {
    k->set = read_env(name, &k->value);
    k->gen = gen;
  }
  return k->set ? k->value : absent;
}

}  // namespace cai4

extern "C" void cascadia_int4_reload_tuning(void) {
  g_gen.fetch_add(1, std::memory_order_acq_rel);
}
