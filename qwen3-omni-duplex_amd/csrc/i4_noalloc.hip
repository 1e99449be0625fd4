// i4_moe_forward for callers that cannot allocate device memory (code under
// hipGraph capture, tight serving loops): the workspace is a file-scope device
// array of fixed size instead of caller memory.
//
// Each GPU the library runs on holds its own copy of `scratch` until the
// process ends.  Its device address is looked up once per device with that
// device current (hipGetSymbolAddress) and kept; the host-side name of the
// array is never handed to a kernel.  Every call on one GPU shares that GPU's
// array: calls that overlap on a GPU (two streams, two host threads) race and
// must be serialised by the caller.  Nothing in the array needs to be zero
// before a call: the MoE pipeline writes every word it reads first (the decode
// layer's pending activation pattern and the status word are written by its
// first kernel).
#include <hip/hip_runtime.h>

#include <mutex>

#include "i4moe.h"
#include "i4_launch.h"

static __device__ __align__(256) unsigned char scratch[I4_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kMaxDevices = 64;
void* g_scratch[kMaxDevices];  // device address of `scratch` on each device, once looked up
std::mutex g_mutex;

// device address of this device's copy of `scratch` (dev is the stream's device)
int scratch_on(int dev, void** out) {
  if (dev < 0 || dev >= kMaxDevices) return I4_ERR_LAUNCH;
  std::lock_guard<std::mutex> lock(g_mutex);
  if (!g_scratch[dev]) {
    int cur = -1;
    if (hipGetDevice(&cur) != hipSuccess) return I4_ERR_LAUNCH;
    if (cur != dev && hipSetDevice(dev) != hipSuccess) return I4_ERR_LAUNCH;
    void* p = nullptr;
    const hipError_t rc = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (cur != dev) (void)hipSetDevice(cur);
    if (rc != hipSuccess || !p) return I4_ERR_LAUNCH;
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return I4_OK;
}

}  // namespace

extern "C" {

int i4_moe_forward_noalloc(const void* x, int x_dtype, int T, const i4_moe_weights* weights,
                           int topk, int renorm, const void* logits, const void* residual,
                           void* out, int32_t* sel_out, float* w_out, int32_t* status_out,
                           hipStream_t stream) {
  if (!weights) return I4_ERR_NULL;
  const size_t need = i4_moe_workspace_bytes(T, weights->gate_up.K, weights->down.K,
                                             weights->gate_up.E, topk);
  if (need == 0) return I4_ERR_SHAPE;
  if (need > (size_t)I4_NOALLOC_SCRATCH_BYTES) return I4_ERR_SCRATCH;
  int dev = -1;
  if (stream) {
    if (hipStreamGetDevice(stream, &dev) != hipSuccess) return I4_ERR_LAUNCH;
  } else if (hipGetDevice(&dev) != hipSuccess) {
    return I4_ERR_LAUNCH;
  }
  void* ws = nullptr;
  const int rc = scratch_on(dev, &ws);
  if (rc) return rc;
  // the status word goes to status_out when given (the scratch's own copy is not
  // reachable by the caller)
  return i4::moe_forward_status(x, x_dtype, T, weights, topk, renorm, logits, residual, out,
                                 sel_out, w_out, ws, (size_t)I4_NOALLOC_SCRATCH_BYTES,
                                 status_out, stream);
}

}  // extern "C"
