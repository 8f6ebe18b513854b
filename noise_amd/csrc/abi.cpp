// Error state, version and launch timing of the C ABI.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>
#include <vector>

#include "common.h"

static thread_local char g_error[1024] = "";

int noise_set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

extern "C" const char* noise_last_error(void) { return g_error; }

extern "C" int noise_abi_version(void) { return 5; }

// ---- timing -----------------------------------------------------------------------------------------------------
namespace {
struct Pending { int cls; hipEvent_t start, stop; };
std::mutex g_mu;
bool g_timing = false;
std::vector<Pending> g_pending;
std::vector<hipEvent_t> g_free;
const char* kNames[kTimeClasses] = {"noise", "embed", "norm", "qkv_gemm", "rope_norm", "attention", "attn_proj_gemm",
                                    "fc_gemm", "rowdot", "mlp_proj_gemm", "head_ce_gemm", "ce_finalize", "credit_lse",
                                    "credit_value", "outer_grad", "lowrank_gemm", "credit_center",
                                    "head_error", "dust_rerun", "dust_errors", "lowrank_pre", "lowrank_post", "fitness", "vector_grad", "adamw",
                                    "reassemble", "linear"};
int64_t g_count[kTimeClasses];
double g_ms[kTimeClasses];

hipEvent_t take_event() {
  if (!g_free.empty()) { hipEvent_t e = g_free.back(); g_free.pop_back(); return e; }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}
}  // namespace

NoiseTimer::NoiseTimer(int cls, hipStream_t s) : slot(-1), stream(s) {
  if (cls < 0) return;  // an untimed launch (the no-allocation entry points create no events)
  std::lock_guard<std::mutex> lk(g_mu);
  if (!g_timing) return;
  Pending p{cls, take_event(), take_event()};
  if (!p.start || !p.stop) return;
  if (hipEventRecord(p.start, s) != hipSuccess) return;
  g_pending.push_back(p);
  slot = (int)g_pending.size() - 1;
}

NoiseTimer::~NoiseTimer() {
  if (slot < 0) return;
  std::lock_guard<std::mutex> lk(g_mu);
  if (slot < (int)g_pending.size()) (void)hipEventRecord(g_pending[slot].stop, stream);
}

// Enables (1) or disables (0) launch timing; enabling clears the accumulated figures.
extern "C" int noise_timing_enable(int enable) {
  std::lock_guard<std::mutex> lk(g_mu);
  g_timing = enable != 0;
  if (g_timing) {
    for (int c = 0; c < kTimeClasses; ++c) { g_count[c] = 0; g_ms[c] = 0.0; }
  }
  return NOISE_OK;
}

// Waits for the recorded launches, folds them into the per-class sums and copies out up to n classes:
// counts[c] launches, total_ms[c] milliseconds, names[c] class names. Returns the number of classes.
extern "C" int noise_timing_read(int32_t n, int64_t* counts, double* total_ms, const char** names) {
  std::lock_guard<std::mutex> lk(g_mu);
  for (auto& p : g_pending) {
    float ms = 0.f;
    if (hipEventSynchronize(p.stop) == hipSuccess && hipEventElapsedTime(&ms, p.start, p.stop) == hipSuccess) {
      g_count[p.cls] += 1;
      g_ms[p.cls] += ms;
    }
    g_free.push_back(p.start);
    g_free.push_back(p.stop);
  }
  g_pending.clear();
  for (int c = 0; c < n && c < kTimeClasses; ++c) {
    if (counts) counts[c] = g_count[c];
    if (total_ms) total_ms[c] = g_ms[c];
    if (names) names[c] = kNames[c];
  }
  return kTimeClasses;
}
