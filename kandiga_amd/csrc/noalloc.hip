// kmoe_forward_noalloc: the routed layer with the library's own static scratch as workspace, for
// callers that cannot allocate device memory (code under HIP graph capture, tight serving loops,
// harnesses that forbid hipMalloc).
//
// The scratch is one file-scope __device__ array per GPU the library runs on, held until the
// process ends.  Host code never passes the array's name to a kernel (on the host it is only a
// stand-in for the symbol): the first call on each device, with that device current, looks up
// the array's device address with hipGetSymbolAddress and keeps it per device; every call then
// hands that address to the kernels as their workspace.  The call allocates nothing itself:
// the forward path it shares with kmoe_forward only carves the given workspace and launches.
//
// All calls on one GPU share its array, which keeps the last call's contents; calls that overlap
// on one GPU (several host threads, or several streams at once) race on it.  Nothing in it has
// to start at zero: the kernels rewrite every word they read before reading it, and the device
// error flags (the only word accumulated across calls) cannot be read through this entry point.
#include <mutex>

#include "../../include/kandiga_amd.h"
#include "kmoe_internal.h"

namespace {

constexpr size_t KMOE_NOALLOC_SCRATCH = (size_t)KMOE_NOALLOC_SCRATCH_BYTES;
static_assert(KMOE_NOALLOC_SCRATCH % 256 == 0, "scratch size must keep 256-byte alignment");

__device__ __align__(256) uint8_t scratch[KMOE_NOALLOC_SCRATCH];

constexpr int MAX_DEVICES = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[MAX_DEVICES];  // device address of `scratch` on each device, once looked up

// Device address of the current device's scratch (looked up once per device).
int scratch_for_current_device(void** ptr) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return kmoe::report_error(KMOE_ERR_HIP, "hipGetDevice failed");
  if (dev < 0 || dev >= MAX_DEVICES) return kmoe::report_error(KMOE_ERR_UNSUPPORTED, "device ordinal out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return kmoe::report_error(KMOE_ERR_HIP, "hipGetSymbolAddress of the static scratch failed");
    g_scratch_ptr[dev] = p;
  }
  *ptr = g_scratch_ptr[dev];
  return KMOE_OK;
}

}  // namespace

extern "C" int kmoe_forward_noalloc(const kmoe_layer* layer, const void* x, const float* logits, int32_t tokens,
                                    void* out, int32_t out_dtype, int32_t* idx_out, float* weights_out,
                                    void* stream) {
  if (!layer) return kmoe::report_error(KMOE_ERR_INVALID_ARG, "null layer");
  if (tokens < 0) return kmoe::report_error(KMOE_ERR_INVALID_ARG, "tokens must be >= 0");
  size_t need = 0;
  int rc = kmoe::workspace_bytes_for(layer, tokens, &need);
  if (rc != KMOE_OK) return rc;
  if (need > KMOE_NOALLOC_SCRATCH) {
    char msg[160];
    snprintf(msg, sizeof msg, "kmoe_forward_noalloc: %d tokens need %zu bytes of scratch, the static scratch holds %zu",
             (int)tokens, need, KMOE_NOALLOC_SCRATCH);
    return kmoe::report_error(KMOE_ERR_WORKSPACE, msg);
  }
  void* ws = nullptr;
  if ((rc = scratch_for_current_device(&ws)) != KMOE_OK) return rc;
  return kmoe::forward_impl(layer, x, logits, tokens, out, out_dtype, idx_out, weights_out, ws, KMOE_NOALLOC_SCRATCH,
                            stream);
}
