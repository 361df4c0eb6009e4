// Allocation-free layer backward: mhc_layer_bwd with its workspace in a
// fixed device array instead of a caller buffer.
//
// The array lives in this file only, so its storage (kScratchBytes per GPU)
// is reserved when this file's code object is loaded on a device, which
// happens at the first mhc_layer_bwd_noalloc call there, and is held until
// the process ends.  Every call on one GPU uses that GPU's copy and leaves
// its contents behind: nothing in the workspace has to start at zero (each
// partial row, the second-stage rows and the Sinkhorn VJP state are written
// in full before they are read), so no clearing is needed between calls.
// Calls that overlap on one GPU (different streams, or threads using
// different streams) race on the array; calls on one stream are ordered by
// the stream.
#include <mutex>

#include "mhc_host.hpp"

namespace {

constexpr size_t kScratchBytes = size_t(64) << 20;
constexpr int kScratchDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kScratchDevices] = {};

// Device address of this device's copy of `scratch`, looked up once per
// device with that device current.  The array's host-side name is only a
// registration handle: kernels must be given this address.
int scratch_address(void** out) {
  int dev = -1;
  MHC_CHECK_HIP(hipGetDevice(&dev));
  MHC_CHECK_ARG(dev >= 0 && dev < kScratchDevices, "device %d is outside the %d devices served", dev,
                kScratchDevices);
  std::lock_guard<std::mutex> lk(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    MHC_CHECK_HIP(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)));
    MHC_CHECK_ARG(p != nullptr, "hipGetSymbolAddress returned NULL for the scratch array");
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return MHC_OK;
}

}  // namespace

extern "C" int mhc_layer_bwd_noalloc(const void* x, int x_dtype, const void* dout, int dout_dtype,
                                     const float* h_pre_raw, const float* h_post_raw, const float* h_res_raw,
                                     const float* M, const float* rms_weight, void* dx, float* d_h_pre_raw,
                                     float* d_h_post_raw, float* d_h_res_raw, float* d_rms_weight, int64_t T,
                                     int n, int C, int per_token, int iters, float eps, void* stream) {
  mhc::clear_error();
  MHC_CHECK_ARG(n >= 1 && n <= MHC_MAX_N, "n=%d must be in [1, %d]", n, MHC_MAX_N);
  MHC_CHECK_ARG(C >= 1, "C=%d must be positive", C);
  MHC_CHECK_ARG(T >= 0, "T=%lld must be >= 0", (long long)T);
  MHC_CHECK_ARG(iters >= 0, "iters=%d must be >= 0", iters);
  const size_t need = mhc_layer_bwd_workspace_bytes(T > 0 ? T : 1, n, C, per_token, iters);
  MHC_CHECK_ARG(need <= kScratchBytes,
                "T=%lld n=%d C=%d needs %zu bytes of workspace, more than the %zu bytes of "
                "mhc_layer_bwd_noalloc's fixed array; call mhc_layer_bwd with a workspace",
                (long long)T, n, C, need, kScratchBytes);
  void* ws = nullptr;
  const int rc = scratch_address(&ws);
  if (rc != MHC_OK) return rc;
  return mhc_layer_bwd(x, x_dtype, dout, dout_dtype, h_pre_raw, h_post_raw, h_res_raw, M, rms_weight, dx,
                       d_h_pre_raw, d_h_post_raw, d_h_res_raw, d_rms_weight, ws, kScratchBytes, T, n, C, per_token,
                       iters, eps, stream);
}
