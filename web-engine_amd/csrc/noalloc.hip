// Kernel scratch of the allocation-free entry point (we_matmul_noalloc): one file-scope device array per GPU, so a
// call needs no hipMalloc. The array holds the split-K partial sums of small-M GEMMs; each slice of a launch
// writes every value of its partial-sum plane before the reduce pass reads it, so nothing has to start at zero
// and the contents a previous call left behind are never read. Every call on one GPU shares that GPU's array, so
// calls that overlapped on one GPU would race: the array belongs to one live context at a time (the first to call,
// until it is destroyed), and the runtime refuses calls from any other context and from a context's second compute
// stream.
#include <mutex>

#include "internal.h"

namespace we {

namespace {

static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_ptr[kMaxDevices] = {};  // device address of `scratch` on each GPU (each holds its own copy)
const void* g_owner[kMaxDevices] = {};  // the context that holds each GPU's array, or null

}  // namespace

hipError_t noalloc_scratch_init(int device) {
  if (device < 0 || device >= kMaxDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_ptr[device]) return hipSuccess;
  int cur = -1;
  hipError_t e = hipGetDevice(&cur);
  if (e != hipSuccess) return e;
  if (cur != device) return hipErrorInvalidDevice;  // the caller makes `device` current first
  void* p = nullptr;
  e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  g_ptr[device] = p;
  return hipSuccess;
}

void* noalloc_scratch(int device) {
  if (device < 0 || device >= kMaxDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_mu);
  return g_ptr[device];
}

bool noalloc_claim(int device, const void* owner) {
  if (device < 0 || device >= kMaxDevices || !owner) return false;
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_owner[device]) g_owner[device] = owner;
  return g_owner[device] == owner;
}

void noalloc_release(int device, const void* owner) {
  if (device < 0 || device >= kMaxDevices) return;
  std::lock_guard<std::mutex> lock(g_mu);
  if (g_owner[device] == owner) g_owner[device] = nullptr;
}

}  // namespace we
