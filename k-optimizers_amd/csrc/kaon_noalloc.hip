// kaon_noalloc.hip -- the allocation-free Adakaon step.
//
// kaon_adakaon_step takes its workspace (per-row / per-column / per-block
// intermediates, the clip divisor, the cautious keep count) from the caller,
// who allocates it with the plan.  Callers that cannot allocate device memory
// at all -- code under HIP graph capture, tight serving loops, harnesses that
// forbid hipMalloc -- call kaon_adakaon_step_noalloc instead: the same kernels,
// with the workspace taken from `scratch`, a file-scope device array of
// KAON_NOALLOC_WS_BYTES that every device holds from module load until the
// process ends.
//
// `scratch` names a host-side stand-in in host code, not a device address.
// Its address on a device comes from hipGetSymbolAddress with that device
// current; it is looked up once per device (on the first call there) and kept
// in `g_scratch`.  Only that address is ever passed to a kernel.
//
// Every call on a device shares the device's array, which keeps the previous
// call's contents.  The step rewrites everything it reads before reading it
// (phase 1 clears the keep count and the 4-bit block maxima), so no clearing
// is needed between calls; calls that overlap on one device (two streams, two
// host threads) race on the array.
#include <hip/hip_runtime.h>

#include <cstdint>
#include <mutex>
#include <string>

#include "kaon_amd.h"

void kaon_set_error(const std::string& s);

namespace {

constexpr int kMaxDevices = 64;

__device__ __align__(256) float scratch[KAON_NOALLOC_WS_BYTES / sizeof(float)];

std::mutex g_scratch_mu;
void* g_scratch[kMaxDevices] = {};

int noalloc_fail(const std::string& s, hipError_t e = hipSuccess) {
  std::string msg = s;
  if (e != hipSuccess) {
    msg += ": ";
    msg += hipGetErrorString(e);
  }
  kaon_set_error(msg);
  return e != hipSuccess ? (int)e : -1;
}

// Device address of `scratch` on the current device.
int scratch_here(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return noalloc_fail("kaon_adakaon_step_noalloc: hipGetDevice", e);
  if (dev < 0 || dev >= kMaxDevices) return noalloc_fail("kaon_adakaon_step_noalloc: device index out of range");
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return noalloc_fail("kaon_adakaon_step_noalloc: hipGetSymbolAddress(scratch)", e);
    if (!p || ((uintptr_t)p % 256) != 0)
      return noalloc_fail("kaon_adakaon_step_noalloc: the static workspace has no 256-byte aligned address");
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return 0;
}

}  // namespace

extern "C" int kaon_adakaon_step_noalloc(const KaonLaunch* L, const KaonHyper* hp, void* stream) {
  if (!L || !hp) return noalloc_fail("kaon_adakaon_step_noalloc: null argument");
  const int64_t cap = (int64_t)(KAON_NOALLOC_WS_BYTES / sizeof(float));
  const int64_t need = L->ws_words;
  if (L->n_tensors > 0 && need <= 0)
    return noalloc_fail("kaon_adakaon_step_noalloc: the launch carries no workspace size (KaonLaunch.ws_words, "
                        "the plan's KaonPlanInfo.ws_words)");
  if (need > cap)
    return noalloc_fail("kaon_adakaon_step_noalloc: the plan needs a workspace of " + std::to_string(need) +
                        " words; the static workspace holds " + std::to_string(cap) +
                        " (KAON_NOALLOC_WS_BYTES); step this group with kaon_adakaon_step");
  void* ws = nullptr;
  const int rc = scratch_here(&ws);
  if (rc) return rc;
  KaonLaunch l = *L;
  l.workspace = ws;
  l.n_long = 0;  // a torch-order step on the caller's stream alone: the side stream would be created here
  return kaon_adakaon_step(&l, hp, stream);
}
