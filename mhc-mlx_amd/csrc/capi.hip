// C ABI plumbing: version, per-thread error text, the launch-shape knob
// table, cached device properties.
#include <climits>
#include <atomic>
#include <mutex>
#include <unordered_map>

#include "mhc_host.hpp"
#include "mhc_plan.hpp"

namespace mhc {

namespace {
thread_local char g_error[1024] = {0};
constexpr int kMaxDevices = 64;
std::atomic<int> g_cus[kMaxDevices];

struct OccKey {
  const void* fn;
  int tpb;
  size_t smem;
  int dev;
  bool operator==(const OccKey& o) const {
    return fn == o.fn && tpb == o.tpb && smem == o.smem && dev == o.dev;
  }
};
struct OccHash {
  size_t operator()(const OccKey& k) const {
    return std::hash<const void*>()(k.fn) ^ (std::hash<int>()(k.tpb) * 31) ^
           (std::hash<size_t>()(k.smem) * 131) ^ (std::hash<int>()(k.dev) * 7);
  }
};
std::mutex g_occ_mu;
std::unordered_map<OccKey, int, OccHash> g_occ;
}  // namespace

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int device_cu_count() {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) dev = 0;
  int v = g_cus[dev].load(std::memory_order_relaxed);
  if (v > 0) return v;
  int cus = 0;
  if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0)
    cus = 1;
  g_cus[dev].store(cus, std::memory_order_relaxed);
  return cus;
}

int occupancy_blocks(const void* kernel, int tpb, size_t smem) {
  int dev = 0;
  (void)hipGetDevice(&dev);
  const OccKey key{kernel, tpb, smem, dev};
  {
    std::lock_guard<std::mutex> lk(g_occ_mu);
    auto it = g_occ.find(key);
    if (it != g_occ.end()) return it->second;
  }
  int blocks = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&blocks, kernel, tpb, smem) != hipSuccess)
    blocks = 0;
  std::lock_guard<std::mutex> lk(g_occ_mu);
  g_occ[key] = blocks;
  return blocks;
}

// ---------------------------------------------------------------------------
// Knobs: one process-wide table of integer launch-shape choices.  Each entry
// starts from its environment variable, read once when the library is
// loaded (static initialisation, before any thread can launch); afterwards
// only mhc_set_knob / mhc_unset_knob change it.  Values are atomics, so a
// setter racing a launch on another thread is well defined (the launch sees
// the old or the new value).  INT_MIN marks an unset knob.
// ---------------------------------------------------------------------------

namespace {
constexpr int kUnset = INT_MIN;
const char* const kKnobNames[kNumKnobs] = {
    "MHC_FWD_MFMA", "MHC_FWD_SPW", "MHC_FWD_CH", "MHC_FWD_TPB", "MHC_FWD_GRID", "MHC_FWD_SKF",
    "MHC_BWD_GRID", "MHC_BWD_MFMA", "MHC_BWD_SPW", "MHC_BWD_LEGACY", "MHC_BWD_TPB",
    "MHC_SK16", "MHC_SK16_CPL", "MHC_SK16_RECORD",
    "MHC_RES_GRID", "MHC_MIX_FWD_GRID", "MHC_MIX_BWD_GRID", "MHC_SCALE_FWD_GRID", "MHC_SCALE_BWD_GRID",
    "MHC_BWD_PIPE", "MHC_MIX32", "MHC_MF32_WAVES", "MHC_SK_BLK_RECORD", "MHC_MF32_FWD_LOOP",
    "MHC_MF32_FWD_WAVES", "MHC_FWD_PIPE", "MHC_SCALE_FWD_FLAT", "MHC_SCALE_BWD_FLAT", "MHC_GEN_MFMA",
    "MHC_SK_WG",
};
std::atomic<int> g_knobs[kNumKnobs];

int knob_index(const char* name) {
  if (name == nullptr) return -1;
  for (int i = 0; i < kNumKnobs; ++i)
    if (strcmp(name, kKnobNames[i]) == 0) return i;
  return -1;
}

struct KnobInit {
  KnobInit() {
    for (int i = 0; i < kNumKnobs; ++i) {
      const char* v = getenv(kKnobNames[i]);
      g_knobs[i].store(v != nullptr && *v != '\0' ? atoi(v) : kUnset, std::memory_order_relaxed);
    }
  }
} g_knob_init;
}  // namespace

int knob(Knob k, int dflt) {
  const int v = g_knobs[k].load(std::memory_order_relaxed);
  return v == kUnset ? dflt : v;
}

}  // namespace mhc

extern "C" int mhc_knob_count(void) { return mhc::kNumKnobs; }

extern "C" const char* mhc_knob_name(int index) {
  return index >= 0 && index < mhc::kNumKnobs ? mhc::kKnobNames[index] : nullptr;
}

extern "C" int mhc_set_knob(const char* name, int value) {
  mhc::clear_error();
  const int i = mhc::knob_index(name);
  MHC_CHECK_ARG(i >= 0, "unknown knob %s", name ? name : "(null)");
  MHC_CHECK_ARG(value != mhc::kUnset, "knob value %d is reserved", value);
  mhc::g_knobs[i].store(value, std::memory_order_relaxed);
  return MHC_OK;
}

extern "C" int mhc_unset_knob(const char* name) {
  mhc::clear_error();
  const int i = mhc::knob_index(name);
  MHC_CHECK_ARG(i >= 0, "unknown knob %s", name ? name : "(null)");
  mhc::g_knobs[i].store(mhc::kUnset, std::memory_order_relaxed);
  return MHC_OK;
}

extern "C" int mhc_get_knob(const char* name, int* value) {
  mhc::clear_error();
  const int i = mhc::knob_index(name);
  MHC_CHECK_ARG(i >= 0, "unknown knob %s", name ? name : "(null)");
  const int v = mhc::g_knobs[i].load(std::memory_order_relaxed);
  if (v == mhc::kUnset) return 0;
  if (value != nullptr) *value = v;
  return 1;
}

extern "C" int mhc_abi_version(void) { return MHC_ABI_VERSION; }

extern "C" const char* mhc_last_error(void) { return mhc::g_error; }
