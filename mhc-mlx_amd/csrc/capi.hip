// C ABI plumbing: version, per-thread error text, cached device queries.
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

int env_int(const char* name, int dflt) {
  const char* v = getenv(name);
  if (v == nullptr || *v == '\0') return dflt;
  return atoi(v);
}

}  // namespace mhc

extern "C" int mhc_abi_version(void) { return MHC_ABI_VERSION; }

extern "C" const char* mhc_last_error(void) { return mhc::g_error; }
