// C-ABI runtime of the gfx950 matmul path: context (device, compute + copy streams, events), a pooled
// device-buffer allocator with zero-on-alloc (the semantics of the reference's Graph, src/gpu/graph.ts),
// pinned host memory and ticketed copies for weight streaming, argument validation, and the op entry
// points that hand off to the kernels.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/we.h"
#include "internal.h"

namespace {

constexpr size_t kTicketRing = 1024;

struct Alloc {
  size_t size;  // bytes allocated (a multiple of 256)
  size_t req;   // bytes the caller asked for, rounded up to 4 like the reference's Graph.buffer
};

}  // namespace

struct we_ctx {
  int device = 0;
  hipStream_t compute = nullptr, copy = nullptr;
  hipEvent_t t0 = nullptr, t1 = nullptr;
  std::string err;
  std::map<uintptr_t, Alloc> allocs;                      // every device allocation, by base address
  std::unordered_map<size_t, std::vector<void*>> pool;    // freed buffers by rounded size
  std::vector<void*> owned;                               // live buffers, in creation order (for mark/release)
  std::map<uintptr_t, size_t> pinned;                     // pinned host allocations
  uint64_t created = 0, reused = 0, created_bytes = 0;
  std::vector<hipEvent_t> tickets;
  std::atomic<uint64_t> next_ticket{1};  // read by we_ticket_wait from other host threads
  void* scratch = nullptr;  // kernel scratch (split-K partial sums, attention V^T) of the selected compute
  bool capturing = false;   // stream, grown on demand; between we_graph_begin and we_graph_end
  size_t scratch_bytes = 0;
  // two compute streams (default priority): `compute`, `scratch` and `scratch_bytes` are those of lanes[lane];
  // the other lane's scratch waits in lane_scratch until it is selected again
  hipStream_t lanes[2] = {nullptr, nullptr};
  int lane = 0;
  void* lane_scratch[2] = {nullptr, nullptr};
  size_t lane_scratch_bytes[2] = {0, 0};
  hipEvent_t fork_ev = nullptr, join_ev = nullptr;
  hipDeviceProp_t prop{};
  // scratch blocks that captured graphs hold (graph count per block): a replay writes the scratch its capture
  // named, so a block outgrown while a graph holds it is retired instead of freed, and freed when its last
  // graph is destroyed
  std::map<void*, int> scratch_refs;
  std::vector<void*> retired;
  hipError_t noalloc_status = hipErrorNotInitialized;  // the device's allocation-free scratch lookup
  // failure injection: device bytes the context may hold (pool + scratch; 0 = no cap) and the bytes it holds;
  // poison: freed buffers are filled with 0xff bytes (NaN in every float format) on the compute stream
  size_t alloc_cap = 0, held_bytes = 0;
  bool poison = false;
  std::map<void*, size_t> scratch_sizes;  // bytes of every scratch block (current, other lane's, retired)
  we::Tuning tune;  // kernel-choice switches (we_set_tuning), from the environment at creation
  std::vector<hipEvent_t> marks;  // timestamp slots (we_timer_mark), created on first use
};

namespace {

// message of the last failed call made without a context (e.g. we_matmul_params_make(NULL, ...)), per thread
thread_local std::string g_no_ctx_err = "no context";

int fail(we_ctx* ctx, int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof buf, fmt, ap);
  va_end(ap);
  if (ctx) ctx->err = buf;
  else g_no_ctx_err = buf;
  return code;
}

}  // namespace

namespace we {
void set_no_ctx_error(const char* msg) { g_no_ctx_err = msg; }
}  // namespace we

namespace {

int hip_fail(we_ctx* ctx, hipError_t e, const char* what) {
  return fail(ctx, WE_EHIP, "%s: %s", what, hipGetErrorString(e));
}

#define HIP_OK(ctx, call, what)                     \
  do {                                              \
    hipError_t e_ = (call);                         \
    if (e_ != hipSuccess) return hip_fail(ctx, e_, what); \
  } while (0)

// hipMalloc under the context's allocation cap (we_set_alloc_cap): a cap reached fails like a full device
hipError_t capped_malloc(we_ctx* ctx, void** p, size_t bytes) {
  if (ctx->alloc_cap && ctx->held_bytes + bytes > ctx->alloc_cap) return hipErrorOutOfMemory;
  const hipError_t e = hipMalloc(p, bytes);
  if (e == hipSuccess) ctx->held_bytes += bytes;
  return e;
}

hipError_t scratch_free(we_ctx* ctx, void* p) {
  auto it = ctx->scratch_sizes.find(p);
  if (it != ctx->scratch_sizes.end()) {
    ctx->held_bytes -= it->second < ctx->held_bytes ? it->second : ctx->held_bytes;
    ctx->scratch_sizes.erase(it);
  }
  return hipFree(p);
}

// Scratch for kernels of this context (split-K partial sums, attention V^T), at least `bytes`. Calls are ordered on the
// compute stream, so one buffer serves them all; growing it waits for the work that may still read it.
int ensure_scratch(we_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->scratch_bytes) return WE_OK;
  if (ctx->capturing)
    return fail(ctx, WE_EINVAL, "scratch must grow to %zu bytes: run the call once before capturing it", bytes);
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  if (ctx->scratch) {
    auto held = ctx->scratch_refs.find(ctx->scratch);
    if (held != ctx->scratch_refs.end() && held->second > 0) {
      ctx->retired.push_back(ctx->scratch);  // a live graph replays into it: keep it until that graph goes
    } else {
      HIP_OK(ctx, hipStreamSynchronize(ctx->compute), "hipStreamSynchronize");
      HIP_OK(ctx, scratch_free(ctx, ctx->scratch), "hipFree scratch");
    }
    ctx->scratch = nullptr;
    ctx->scratch_bytes = 0;
  }
  const size_t want = ((bytes < (16u << 20) ? (16u << 20) : bytes) + 4095) / 4096 * 4096;
  void* p = nullptr;
  const hipError_t e = capped_malloc(ctx, &p, want);
  if (e != hipSuccess) return fail(ctx, WE_ENOMEM, "scratch of %zu bytes: %s%s", want, hipGetErrorString(e),
                                   ctx->alloc_cap ? " (allocation cap set)" : "");
  ctx->scratch_sizes[p] = want;
  ctx->scratch = p;
  ctx->scratch_bytes = want;
  return WE_OK;
}

size_t round_size(size_t bytes) { return ((bytes < 4 ? 4 : bytes) + 255) / 256 * 256; }

// Is [p, p + bytes) inside one device allocation of this context?
int check_span(we_ctx* ctx, const void* p, size_t bytes, const char* name) {
  if (bytes == 0) return WE_OK;
  if (!p) return fail(ctx, WE_EINVAL, "%s is null", name);
  const uintptr_t a = (uintptr_t)p;
  auto it = ctx->allocs.upper_bound(a);
  if (it == ctx->allocs.begin()) return fail(ctx, WE_EINVAL, "%s is not a buffer of this context", name);
  --it;
  const uintptr_t base = it->first, end = base + it->second.req;
  if (a >= base + it->second.size) return fail(ctx, WE_EINVAL, "%s is not a buffer of this context", name);
  if (a >= end || bytes > end - a)
    return fail(ctx, WE_EINVAL, "%s is too small: needs %zu bytes at offset %zu of a %zu-byte buffer", name, bytes,
                (size_t)(a - base), it->second.req);
  return WE_OK;
}

int elem_bytes(int dt) {
  switch (dt) {
    case WE_F32: return 4;
    case WE_F16:
    case WE_BF16: return 2;
    case WE_FP8_E4M3: return 1;
    default: return 0;
  }
}

bool is_act(int dt) { return dt == WE_F32 || dt == WE_F16 || dt == WE_BF16; }

hipEvent_t& ticket_event(we_ctx* ctx, uint64_t t) { return ctx->tickets[t % kTicketRing]; }

int new_ticket(we_ctx* ctx, hipStream_t s, uint64_t* out) {
  const uint64_t t = ctx->next_ticket++;
  hipEvent_t& ev = ticket_event(ctx, t);
  HIP_OK(ctx, hipEventRecord(ev, s), "hipEventRecord");
  *out = t;
  return WE_OK;
}

int ticket_valid(we_ctx* ctx, uint64_t t) {
  if (t == 0 || t >= ctx->next_ticket) return fail(ctx, WE_EINVAL, "unknown ticket %llu", (unsigned long long)t);
  if (t + kTicketRing < ctx->next_ticket)
    return fail(ctx, WE_EINVAL, "ticket %llu expired (more than %zu tickets since)", (unsigned long long)t, kTicketRing);
  return WE_OK;
}

}  // namespace

namespace we {
// The switches as the WE_* environment variables give them (the values of sweeps and tests that pin a kernel):
// WE_GEMM_CFG=<id>, WE_GEMM_PATH=generic, WE_GEMM_SPLITK=off|<slices>, WE_GEMM_REDUCE_XCD=off,
// WE_ATTN_PATH=registers|ring|mfma16, WE_INT4_PATH=generic|shared|pipe. Unset or unknown values keep the defaults.
Tuning tuning_from_env() {
  Tuning t;
  auto env = [](const char* name) -> const char* {
    const char* v = getenv(name);
    return v && *v ? v : nullptr;
  };
  if (const char* v = env("WE_GEMM_CFG")) t.gemm_cfg = atoi(v);
  if (const char* v = env("WE_GEMM_PATH")) t.gemm_generic = strcmp(v, "generic") == 0;
  if (const char* v = env("WE_GEMM_SPLITK")) {
    const long n = strtol(v, nullptr, 10);
    t.gemm_splitk = strcmp(v, "off") == 0 ? 0 : n > 0 ? (int)n : -1;
  }
  if (const char* v = env("WE_GEMM_REDUCE_XCD")) t.gemm_reduce_xcd = strcmp(v, "off") != 0;
  if (const char* v = env("WE_ATTN_PATH"))
    t.attn_path = strcmp(v, "registers") == 0 ? 1 : strcmp(v, "ring") == 0 ? 2 : strcmp(v, "mfma16") == 0 ? 3 : 0;
  if (const char* v = env("WE_INT4_PATH"))
    t.int4_path = strcmp(v, "generic") == 0 ? 1 : strcmp(v, "shared") == 0 ? 2 : strcmp(v, "pipe") == 0 ? 3 : 0;
  return t;
}
}  // namespace we

extern "C" {

int we_host_span(we_ctx* ctx, const void* p, size_t bytes);

int we_ctx_create(int device, we_ctx** out) {
  if (!out) return fail(nullptr, WE_EINVAL, "output pointer is null");
  *out = nullptr;
  int count = 0;
  if (hipGetDeviceCount(&count) != hipSuccess || count == 0) return fail(nullptr, WE_EHIP, "no HIP device is visible");
  if (device < 0 || device >= count) return fail(nullptr, WE_EINVAL, "device %d out of range (%d visible)", device, count);
  we_ctx* ctx = new we_ctx();
  ctx->device = device;
  ctx->tune = we::tuning_from_env();
  auto cleanup = [&](int code) {
    we_ctx_destroy(ctx);
    return fail(nullptr, code, "HIP set-up of device %d failed", device);
  };
  if (hipSetDevice(device) != hipSuccess) return cleanup(WE_EHIP);
  if (hipGetDeviceProperties(&ctx->prop, device) != hipSuccess) return cleanup(WE_EHIP);
  // the allocation-free entry point's scratch array on this device (kept per device; its failure is reported by
  // we_matmul_noalloc, the only user)
  ctx->noalloc_status = we::noalloc_scratch_init(device);
  for (auto& st : ctx->lanes)
    if (hipStreamCreateWithFlags(&st, hipStreamNonBlocking) != hipSuccess) return cleanup(WE_EHIP);
  ctx->compute = ctx->lanes[0];
  if (hipStreamCreateWithFlags(&ctx->copy, hipStreamNonBlocking) != hipSuccess) return cleanup(WE_EHIP);
  if (hipEventCreateWithFlags(&ctx->fork_ev, hipEventDisableTiming) != hipSuccess ||
      hipEventCreateWithFlags(&ctx->join_ev, hipEventDisableTiming) != hipSuccess)
    return cleanup(WE_EHIP);
  if (hipEventCreate(&ctx->t0) != hipSuccess || hipEventCreate(&ctx->t1) != hipSuccess) return cleanup(WE_EHIP);
  ctx->tickets.resize(kTicketRing, nullptr);
  for (auto& e : ctx->tickets)
    if (hipEventCreateWithFlags(&e, hipEventDisableTiming) != hipSuccess) return cleanup(WE_EHIP);
  *out = ctx;
  return WE_OK;
}

int we_ctx_destroy(we_ctx* ctx) {
  if (!ctx) return WE_OK;
  (void)hipSetDevice(ctx->device);
  if (ctx->capturing) {
    hipGraph_t g = nullptr;
    if (hipStreamEndCapture(ctx->compute, &g) == hipSuccess && g) (void)hipGraphDestroy(g);
    ctx->capturing = false;
  }
  for (auto st : ctx->lanes)
    if (st) (void)hipStreamSynchronize(st);
  if (ctx->copy) (void)hipStreamSynchronize(ctx->copy);
  we::noalloc_release(ctx->device, ctx);  // its calls are done: another context may take the array
  for (auto& kv : ctx->allocs) (void)hipFree((void*)kv.first);
  if (ctx->scratch) (void)hipFree(ctx->scratch);
  if (ctx->lane_scratch[1 - ctx->lane]) (void)hipFree(ctx->lane_scratch[1 - ctx->lane]);
  for (void* p : ctx->retired) (void)hipFree(p);
  for (auto& kv : ctx->pinned) (void)hipHostFree((void*)kv.first);
  for (auto& e : ctx->tickets)
    if (e) (void)hipEventDestroy(e);
  if (ctx->t0) (void)hipEventDestroy(ctx->t0);
  if (ctx->t1) (void)hipEventDestroy(ctx->t1);
  for (auto& e : ctx->marks)
    if (e) (void)hipEventDestroy(e);
  if (ctx->fork_ev) (void)hipEventDestroy(ctx->fork_ev);
  if (ctx->join_ev) (void)hipEventDestroy(ctx->join_ev);
  for (auto st : ctx->lanes)
    if (st) (void)hipStreamDestroy(st);
  if (ctx->copy) (void)hipStreamDestroy(ctx->copy);
  delete ctx;
  return WE_OK;
}

const char* we_last_error(const we_ctx* ctx) { return ctx ? ctx->err.c_str() : g_no_ctx_err.c_str(); }

int we_set_tuning(we_ctx* ctx, int key, int value, int* previous) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  int* slot = nullptr;
  int lo = 0, hi = 0;
  switch (key) {
    case WE_TUNE_GEMM_CFG: slot = &ctx->tune.gemm_cfg, lo = -1, hi = we::GEMM_CFG_256x192; break;
    case WE_TUNE_GEMM_GENERIC: slot = &ctx->tune.gemm_generic, lo = 0, hi = 1; break;
    case WE_TUNE_GEMM_SPLITK: slot = &ctx->tune.gemm_splitk, lo = -1, hi = 1 << 16; break;
    case WE_TUNE_GEMM_REDUCE_XCD: slot = &ctx->tune.gemm_reduce_xcd, lo = 0, hi = 1; break;
    case WE_TUNE_ATTN_PATH: slot = &ctx->tune.attn_path, lo = 0, hi = 3; break;
    case WE_TUNE_INT4_PATH: slot = &ctx->tune.int4_path, lo = 0, hi = 3; break;
    default: return fail(ctx, WE_EINVAL, "unknown tuning key %d", key);
  }
  if (value < lo || value > hi) return fail(ctx, WE_EINVAL, "tuning key %d takes %d .. %d, got %d", key, lo, hi, value);
  if (previous) *previous = *slot;
  *slot = value;
  return WE_OK;
}

int we_device_info(we_ctx* ctx, char* name, size_t name_len, int* compute_units, int* lds_bytes) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (name && name_len) snprintf(name, name_len, "%s", ctx->prop.gcnArchName);
  if (compute_units) *compute_units = ctx->prop.multiProcessorCount;
  if (lds_bytes) *lds_bytes = (int)ctx->prop.sharedMemPerBlock;
  return WE_OK;
}

// ------------------------------------------------------------------------------------------ buffers

int we_buf_alloc(we_ctx* ctx, size_t bytes, void** out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (!out) return fail(ctx, WE_EINVAL, "output pointer is null");
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  const size_t size = round_size(bytes);
  void* p = nullptr;
  const size_t req = (bytes < 4 ? 4 : (bytes + 3) / 4 * 4);
  auto& list = ctx->pool[size];
  if (!list.empty()) {
    p = list.back();
    list.pop_back();
    ctx->allocs[(uintptr_t)p].req = req;
    ctx->reused++;
  } else {
    hipError_t e = capped_malloc(ctx, &p, size);
    if (e != hipSuccess)
      return fail(ctx, WE_ENOMEM, "hipMalloc(%zu): %s%s", size, hipGetErrorString(e),
                  ctx->alloc_cap ? " (allocation cap set)" : "");
    ctx->allocs[(uintptr_t)p] = Alloc{size, req};
    ctx->created++;
    ctx->created_bytes += size;
  }
  // zeroed like a new WebGPU buffer; a fill kernel rather than a memset node (graph-capture safe)
  hipError_t e = we::launch_zero(p, size, ctx->compute);
  if (e != hipSuccess) return hip_fail(ctx, e, "zero fill");
  ctx->owned.push_back(p);
  *out = p;
  return WE_OK;
}

int we_buf_free(we_ctx* ctx, void* buf) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  auto it = ctx->allocs.find((uintptr_t)buf);
  if (it == ctx->allocs.end()) return fail(ctx, WE_EINVAL, "we_buf_free: not a buffer of this context");
  for (size_t i = 0; i < ctx->owned.size(); i++)
    if (ctx->owned[i] == buf) {
      if (ctx->poison) {
        HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
        const hipError_t e = we::launch_fill(buf, it->second.size, 0xff, ctx->compute);
        if (e != hipSuccess) return hip_fail(ctx, e, "poison fill");
      }
      ctx->owned.erase(ctx->owned.begin() + (long)i);
      ctx->pool[it->second.size].push_back(buf);
      return WE_OK;
    }
  return fail(ctx, WE_EINVAL, "we_buf_free: buffer already freed");
}

int we_buf_upload(we_ctx* ctx, void* buf, size_t offset, const void* src, size_t bytes) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (bytes == 0) return WE_OK;
  if (!src) return fail(ctx, WE_EINVAL, "upload source is null");
  int rc = check_span(ctx, (char*)buf + offset, bytes, "upload destination");
  if (rc) return rc;
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  HIP_OK(ctx, hipMemcpyAsync((char*)buf + offset, src, bytes, hipMemcpyHostToDevice, ctx->compute), "upload");
  HIP_OK(ctx, hipStreamSynchronize(ctx->compute), "upload sync");  // the host copy may be reused on return
  return WE_OK;
}

int we_buf_download(we_ctx* ctx, const void* buf, size_t offset, void* dst, size_t bytes) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (bytes == 0) return WE_OK;
  if (!dst) return fail(ctx, WE_EINVAL, "download destination is null");
  int rc = check_span(ctx, (const char*)buf + offset, bytes, "download source");
  if (rc) return rc;
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  HIP_OK(ctx, hipMemcpyAsync(dst, (const char*)buf + offset, bytes, hipMemcpyDeviceToHost, ctx->compute), "download");
  HIP_OK(ctx, hipStreamSynchronize(ctx->compute), "download sync");
  return WE_OK;
}

int we_buf_download_async(we_ctx* ctx, const void* buf, size_t offset, void* pinned_dst, size_t bytes,
                          uint64_t* ticket) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (!ticket) return fail(ctx, WE_EINVAL, "output pointer is null");
  int rc = check_span(ctx, (const char*)buf + offset, bytes, "download source");
  if (rc) return rc;
  rc = we_host_span(ctx, pinned_dst, bytes);
  if (rc) return rc;
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  if (bytes)
    HIP_OK(ctx, hipMemcpyAsync(pinned_dst, (const char*)buf + offset, bytes, hipMemcpyDeviceToHost, ctx->compute),
           "download");
  return new_ticket(ctx, ctx->compute, ticket);
}

int we_ticket_wait(we_ctx* ctx, uint64_t ticket) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  // reads only the ticket's event (created with the context), so another host thread may keep using ctx; the
  // message of a failure goes to the context-free slot of this thread, not to ctx
  if (ticket == 0 || ticket >= ctx->next_ticket)
    return fail(nullptr, WE_EINVAL, "unknown ticket %llu", (unsigned long long)ticket);
  if (ticket + kTicketRing < ctx->next_ticket)
    return fail(nullptr, WE_EINVAL, "ticket %llu expired (more than %zu tickets since)", (unsigned long long)ticket,
                kTicketRing);
  const hipError_t e = hipEventSynchronize(ticket_event(ctx, ticket));
  if (e != hipSuccess) return fail(nullptr, WE_EHIP, "hipEventSynchronize: %s", hipGetErrorString(e));
  return WE_OK;
}

int we_buf_copy(we_ctx* ctx, const void* src, size_t src_offset, void* dst, size_t dst_offset, size_t bytes) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (bytes == 0) return WE_OK;
  int rc = check_span(ctx, (const char*)src + src_offset, bytes, "copy source");
  if (!rc) rc = check_span(ctx, (char*)dst + dst_offset, bytes, "copy destination");
  if (rc) return rc;
  HIP_OK(ctx, hipMemcpyAsync((char*)dst + dst_offset, (const char*)src + src_offset, bytes, hipMemcpyDeviceToDevice,
                             ctx->compute),
         "copy");
  return WE_OK;
}

int we_mark(we_ctx* ctx, size_t* mark) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (!mark) return fail(ctx, WE_EINVAL, "output pointer is null");
  *mark = ctx->owned.size();
  return WE_OK;
}

int we_release(we_ctx* ctx, size_t mark, void* const* keep, size_t n_keep) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (mark > ctx->owned.size()) return fail(ctx, WE_EINVAL, "mark %zu is past the %zu live buffers", mark, ctx->owned.size());
  if (ctx->poison) HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  std::vector<void*> later(ctx->owned.begin() + (long)mark, ctx->owned.end());
  ctx->owned.resize(mark);
  hipError_t e = hipSuccess;
  for (void* b : later) {
    bool kept = false;
    for (size_t i = 0; i < n_keep && !kept; i++) kept = keep[i] == b;
    if (kept) {
      ctx->owned.push_back(b);
      continue;
    }
    const size_t size = ctx->allocs[(uintptr_t)b].size;
    if (ctx->poison && e == hipSuccess) e = we::launch_fill(b, size, 0xff, ctx->compute);
    ctx->pool[size].push_back(b);
  }
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "poison fill");
}

int we_set_alloc_cap(we_ctx* ctx, uint64_t bytes, uint64_t* held) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  ctx->alloc_cap = (size_t)bytes;
  if (held) *held = ctx->held_bytes;
  return WE_OK;
}

int we_set_poison(we_ctx* ctx, int on) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  ctx->poison = on != 0;
  return WE_OK;
}

int we_stats(we_ctx* ctx, uint64_t* created, uint64_t* reused, uint64_t* created_bytes) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (created) *created = ctx->created;
  if (reused) *reused = ctx->reused;
  if (created_bytes) *created_bytes = ctx->created_bytes;
  return WE_OK;
}

int we_sync(we_ctx* ctx) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  HIP_OK(ctx, hipStreamSynchronize(ctx->copy), "copy stream");
  HIP_OK(ctx, hipStreamSynchronize(ctx->lanes[0]), "compute stream");
  HIP_OK(ctx, hipStreamSynchronize(ctx->lanes[1]), "second compute stream");
  return WE_OK;
}

// ------------------------------------------------------------------------------------------ two compute streams

int we_record_all(we_ctx* ctx, uint64_t tickets[3]) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (!tickets) return fail(ctx, WE_EINVAL, "output pointer is null");
  int rc = new_ticket(ctx, ctx->lanes[0], &tickets[0]);
  if (!rc) rc = new_ticket(ctx, ctx->lanes[1], &tickets[1]);
  if (!rc) rc = new_ticket(ctx, ctx->copy, &tickets[2]);
  return rc;
}

int we_stream_select(we_ctx* ctx, int stream) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (stream != 0 && stream != 1) return fail(ctx, WE_EINVAL, "stream must be 0 or 1, got %d", stream);
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (stream == ctx->lane) return WE_OK;
  ctx->lane_scratch[ctx->lane] = ctx->scratch;
  ctx->lane_scratch_bytes[ctx->lane] = ctx->scratch_bytes;
  ctx->scratch = ctx->lane_scratch[stream];
  ctx->scratch_bytes = ctx->lane_scratch_bytes[stream];
  ctx->lane_scratch[stream] = nullptr;
  ctx->lane_scratch_bytes[stream] = 0;
  ctx->compute = ctx->lanes[stream];
  ctx->lane = stream;
  return WE_OK;
}

int we_stream_fork(we_ctx* ctx) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  HIP_OK(ctx, hipEventRecord(ctx->fork_ev, ctx->lanes[0]), "hipEventRecord");
  HIP_OK(ctx, hipStreamWaitEvent(ctx->lanes[1], ctx->fork_ev, 0), "hipStreamWaitEvent");
  return WE_OK;
}

int we_stream_join(we_ctx* ctx) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  HIP_OK(ctx, hipEventRecord(ctx->join_ev, ctx->lanes[1]), "hipEventRecord");
  HIP_OK(ctx, hipStreamWaitEvent(ctx->lanes[0], ctx->join_ev, 0), "hipStreamWaitEvent");
  return WE_OK;
}

// ------------------------------------------------------------------------------------------ pinned host / streaming

int we_host_alloc(we_ctx* ctx, size_t bytes, void** out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (!out) return fail(ctx, WE_EINVAL, "output pointer is null");
  void* p = nullptr;
  hipError_t e = hipHostMalloc(&p, bytes ? bytes : 1, hipHostMallocDefault);
  if (e != hipSuccess) return fail(ctx, WE_ENOMEM, "hipHostMalloc(%zu): %s", bytes, hipGetErrorString(e));
  ctx->pinned[(uintptr_t)p] = bytes;
  *out = p;
  return WE_OK;
}

int we_host_free(we_ctx* ctx, void* ptr) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  auto it = ctx->pinned.find((uintptr_t)ptr);
  if (it == ctx->pinned.end()) return fail(ctx, WE_EINVAL, "we_host_free: not pinned memory of this context");
  HIP_OK(ctx, hipStreamSynchronize(ctx->copy), "copy stream");
  HIP_OK(ctx, hipHostFree(ptr), "hipHostFree");
  ctx->pinned.erase(it);
  return WE_OK;
}

int we_host_span(we_ctx* ctx, const void* p, size_t bytes) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!p) return fail(ctx, WE_EINVAL, "pinned address is null");
  auto it = ctx->pinned.upper_bound((uintptr_t)p);
  if (it == ctx->pinned.begin()) return fail(ctx, WE_EINVAL, "address is not pinned memory of this context");
  --it;
  const uintptr_t a = (uintptr_t)p, end = it->first + it->second;
  if (a >= end && !(a == it->first && bytes == 0))
    return fail(ctx, WE_EINVAL, "address is not pinned memory of this context");
  if (bytes > end - a)
    return fail(ctx, WE_EINVAL, "%zu bytes at offset %zu run past the %zu-byte pinned buffer", bytes,
                (size_t)(a - it->first), it->second);
  return WE_OK;
}

int we_stream_copy(we_ctx* ctx, void* dst, const void* pinned_src, size_t bytes, uint64_t after, uint64_t* ticket) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (!ticket) return fail(ctx, WE_EINVAL, "output pointer is null");
  int rc = check_span(ctx, dst, bytes, "stream destination");
  if (rc) return rc;
  auto it = ctx->pinned.upper_bound((uintptr_t)pinned_src);
  if (it == ctx->pinned.begin()) return fail(ctx, WE_EINVAL, "stream source is not pinned memory of this context");
  --it;
  if ((uintptr_t)pinned_src + bytes > it->first + it->second)
    return fail(ctx, WE_EINVAL, "stream source is not pinned memory of this context");
  if (after) {
    rc = ticket_valid(ctx, after);
    if (rc) return rc;
    HIP_OK(ctx, hipStreamWaitEvent(ctx->copy, ticket_event(ctx, after), 0), "hipStreamWaitEvent");
  }
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  HIP_OK(ctx, hipMemcpyAsync(dst, pinned_src, bytes, hipMemcpyHostToDevice, ctx->copy), "stream copy");
  return new_ticket(ctx, ctx->copy, ticket);
}

int we_wait_ticket(we_ctx* ctx, uint64_t ticket) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  int rc = ticket_valid(ctx, ticket);
  if (rc) return rc;
  HIP_OK(ctx, hipStreamWaitEvent(ctx->compute, ticket_event(ctx, ticket), 0), "hipStreamWaitEvent");
  return WE_OK;
}

int we_record_compute(we_ctx* ctx, uint64_t* ticket) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (!ticket) return fail(ctx, WE_EINVAL, "output pointer is null");
  return new_ticket(ctx, ctx->compute, ticket);
}

int we_ticket_done(we_ctx* ctx, uint64_t ticket, int* done) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (!done) return fail(ctx, WE_EINVAL, "output pointer is null");
  int rc = ticket_valid(ctx, ticket);
  if (rc) return rc;
  hipError_t e = hipEventQuery(ticket_event(ctx, ticket));
  if (e == hipSuccess) *done = 1;
  else if (e == hipErrorNotReady) *done = 0;
  else return hip_fail(ctx, e, "hipEventQuery");
  return WE_OK;
}

struct we_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  void* scratch = nullptr;  // the scratch block the captured kernels name (held until destroy)
  int lane = 0;             // the compute stream it was captured on, and the only one it replays on
};

int we_graph_begin(we_ctx* ctx) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "a graph is already being captured");
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  HIP_OK(ctx, hipStreamBeginCapture(ctx->compute, hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
  ctx->capturing = true;
  return WE_OK;
}

int we_graph_end(we_ctx* ctx, we_graph** graph) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!graph) return fail(ctx, WE_EINVAL, "output pointer is null");
  if (!ctx->capturing) return fail(ctx, WE_EINVAL, "no graph is being captured");
  ctx->capturing = false;
  hipGraph_t g = nullptr;
  HIP_OK(ctx, hipStreamEndCapture(ctx->compute, &g), "hipStreamEndCapture");
  hipGraphExec_t exec = nullptr;
  const hipError_t e = hipGraphInstantiate(&exec, g, nullptr, nullptr, 0);
  if (e != hipSuccess) {
    (void)hipGraphDestroy(g);
    return hip_fail(ctx, e, "hipGraphInstantiate");
  }
  *graph = new we_graph{g, exec, ctx->scratch, ctx->lane};
  if (ctx->scratch) ctx->scratch_refs[ctx->scratch]++;
  return WE_OK;
}

int we_graph_launch(we_ctx* ctx, we_graph* graph) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!graph) return fail(ctx, WE_EINVAL, "graph is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  // its kernels use the scratch of the stream it was captured on, ordered only against that stream's work
  if (graph->lane != ctx->lane)
    return fail(ctx, WE_EINVAL, "graph was captured on compute stream %d; select that stream to launch it", graph->lane);
  HIP_OK(ctx, hipGraphLaunch(graph->exec, ctx->compute), "hipGraphLaunch");
  return WE_OK;
}

int we_graph_destroy(we_ctx* ctx, we_graph* graph) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!graph) return WE_OK;
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  HIP_OK(ctx, hipStreamSynchronize(ctx->lanes[graph->lane]), "hipStreamSynchronize");
  (void)hipGraphExecDestroy(graph->exec);
  (void)hipGraphDestroy(graph->graph);
  if (graph->scratch) {
    auto held = ctx->scratch_refs.find(graph->scratch);
    if (held != ctx->scratch_refs.end() && --held->second <= 0) {
      ctx->scratch_refs.erase(held);
      for (size_t i = 0; i < ctx->retired.size(); i++)
        if (ctx->retired[i] == graph->scratch) {  // outgrown meanwhile and no graph left on it
          (void)scratch_free(ctx, graph->scratch);
          ctx->retired.erase(ctx->retired.begin() + (long)i);
          break;
        }
    }
  }
  delete graph;
  return WE_OK;
}

int we_timer_start(we_ctx* ctx) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  HIP_OK(ctx, hipEventRecord(ctx->t0, ctx->compute), "hipEventRecord");
  return WE_OK;
}

int we_timer_stop(we_ctx* ctx, float* ms) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (!ms) return fail(ctx, WE_EINVAL, "output pointer is null");
  HIP_OK(ctx, hipEventRecord(ctx->t1, ctx->compute), "hipEventRecord");
  HIP_OK(ctx, hipEventSynchronize(ctx->t1), "hipEventSynchronize");
  HIP_OK(ctx, hipEventElapsedTime(ms, ctx->t0, ctx->t1), "hipEventElapsedTime");
  return WE_OK;
}

int we_timer_mark(we_ctx* ctx, uint32_t slot) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->capturing) return fail(ctx, WE_EINVAL, "not allowed while a graph is being captured");
  if (slot >= WE_TIMER_MARKS) return fail(ctx, WE_EINVAL, "timer slot %u out of range (%d slots)", slot, WE_TIMER_MARKS);
  if (ctx->marks.empty()) {
    ctx->marks.assign(WE_TIMER_MARKS, nullptr);
    for (auto& e : ctx->marks) HIP_OK(ctx, hipEventCreate(&e), "hipEventCreate");
  }
  HIP_OK(ctx, hipEventRecord(ctx->marks[slot], ctx->compute), "hipEventRecord");
  return WE_OK;
}

int we_timer_between(we_ctx* ctx, uint32_t from, uint32_t to, float* ms) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!ms) return fail(ctx, WE_EINVAL, "output pointer is null");
  if (ctx->marks.empty() || from >= WE_TIMER_MARKS || to >= WE_TIMER_MARKS)
    return fail(ctx, WE_EINVAL, "timer slots %u, %u were not marked", from, to);
  HIP_OK(ctx, hipEventSynchronize(ctx->marks[to]), "hipEventSynchronize");
  HIP_OK(ctx, hipEventElapsedTime(ms, ctx->marks[from], ctx->marks[to]), "hipEventElapsedTime");
  return WE_OK;
}

// ------------------------------------------------------------------------------------------ matmul

int we_matmul_params_make(we_ctx* ctx, uint32_t m, uint32_t n, uint32_t k, float scale, int64_t x_stride,
                          int64_t w_stride, int64_t y_stride, int64_t x_offset, int64_t w_offset, int64_t y_offset,
                          int64_t k_split, we_matmul_params* out) {
  if (!out) return fail(ctx, WE_EINVAL, "params output is null");
  const int64_t xs = x_stride < 0 ? k : x_stride, ws = w_stride < 0 ? k : w_stride, ys = y_stride < 0 ? n : y_stride;
  const int64_t xo = x_offset < 0 ? 0 : x_offset, wo = w_offset < 0 ? 0 : w_offset, yo = y_offset < 0 ? 0 : y_offset;
  const char* names[5] = {"K", "xStride", "wStride", "xOffset", "wOffset"};
  const int64_t vals[5] = {(int64_t)k, xs, ws, xo, wo};
  for (int i = 0; i < 5; i++)
    if (vals[i] % 4) return fail(ctx, WE_EINVAL, "%s must be a multiple of 4, got %lld", names[i], (long long)vals[i]);
  *out = we_matmul_params{m, n, k, scale, (uint32_t)xs, (uint32_t)ws, (uint32_t)ys, (uint32_t)xo, (uint32_t)wo,
                          (uint32_t)yo, 0, 0, (uint32_t)(k_split < 1 ? 1 : k_split)};
  return WE_OK;
}

int we_conv3x3_params(we_ctx* ctx, uint32_t height, uint32_t width, uint32_t cin, uint32_t cout,
                      we_matmul_params* out) {
  if (!out) return fail(ctx, WE_EINVAL, "params output is null");
  if (cin % 4) return fail(ctx, WE_EINVAL, "cin must be a multiple of 4, got %u", cin);
  const uint32_t m = height * width, k = 9 * cin;
  *out = we_matmul_params{m, cout, k, 1.0f, k, k, cout, 0, 0, 0, width, cin, 1};
  return WE_OK;
}

uint32_t we_ksplit_for(uint32_t m, uint32_t n, uint32_t k) {
  const uint32_t tiles = ((m + 127) / 128) * ((n + 127) / 128);
  const uint32_t want = (256 + tiles - 1) / tiles, cap = k / 256;
  const uint32_t s = want < cap ? want : cap;
  return s < 1 ? 1 : s;
}

namespace {
// the q/k path of attend() fused into a QKV projection (we_matmul_qk_norm_rope)
struct QkFuse {
  uint32_t q_heads, k_heads;
  float eps, offset;
  const float* norm_q;
  const float* norm_k;
  uint32_t rope_from;
  const float* cos_t;
  const float* sin_t;
};

int matmul_impl(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags,
                const float* gate, const void* res, bool noalloc = false, int mul = 0, const QkFuse* qk = nullptr);
}  // namespace

int we_matmul(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
              const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags) {
  return matmul_impl(ctx, p, x_dtype, x, w_dtype, w, w_scales, group, y_dtype, y, bias, flags, nullptr, nullptr);
}

int we_matmul_noalloc(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                      const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (ctx->noalloc_status != hipSuccess)
    return hip_fail(ctx, ctx->noalloc_status, "allocation-free scratch of this device");
  // one fixed array per GPU: a call that could overlap another call's use of it is refused, not raced
  if (ctx->lane != 0)
    return fail(ctx, WE_EINVAL, "we_matmul_noalloc runs on compute stream 0 only (select stream 0): the device's fixed "
                                "scratch array would be shared with the other stream's calls");
  if (!we::noalloc_claim(ctx->device, ctx))
    return fail(ctx, WE_EINVAL, "the allocation-free scratch array of device %d belongs to another live context",
                ctx->device);
  return matmul_impl(ctx, p, x_dtype, x, w_dtype, w, w_scales, group, y_dtype, y, bias, flags, nullptr, nullptr, true);
}

int we_matmul_gated(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                    const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags,
                    const float* gate, const void* residual) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!gate) return fail(ctx, WE_EINVAL, "gate is null");
  if (flags & WE_EPI_SPLIT_K) return fail(ctx, WE_EINVAL, "a gated residual does not combine with split-K partials");
  if (residual && (flags & WE_EPI_ACCUMULATE))
    return fail(ctx, WE_EINVAL, "a residual replaces accumulate: pass y as the residual to add to y");
  return matmul_impl(ctx, p, x_dtype, x, w_dtype, w, w_scales, group, y_dtype, y, bias, flags, gate, residual);
}

int we_matmul_mul(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                  const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags, int mul,
                  const void* aux) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (mul != WE_MUL_SWIGLU && mul != WE_MUL_SIGMOID_GATE) return fail(ctx, WE_EINVAL, "unknown product epilogue %d", mul);
  if (!aux) return fail(ctx, WE_EINVAL, "aux is null");
  if (flags & (WE_EPI_ACCUMULATE | WE_EPI_SPLIT_K | WE_EPI_GELU_TANH))
    return fail(ctx, WE_EINVAL, "a product epilogue takes only WE_EPI_BIAS (flags 0x%x)", flags);
  if (w_dtype == WE_INT4) return fail(ctx, WE_EUNSUPPORTED, "int4 weights have no product epilogue");
  return matmul_impl(ctx, p, x_dtype, x, w_dtype, w, w_scales, group, y_dtype, y, bias, flags, nullptr, aux, false,
                     mul);
}

int we_matmul_qk_norm_rope(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype,
                           const void* w, int y_dtype, void* y, const float* bias, uint32_t flags, uint32_t q_heads,
                           uint32_t k_heads, float eps, float offset, const float* norm_q, const float* norm_k,
                           uint32_t rope_from, const float* cos_t, const float* sin_t) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!p) return fail(ctx, WE_EINVAL, "params is null");
  if (flags & ~WE_EPI_BIAS) return fail(ctx, WE_EINVAL, "the fused q/k projection takes only WE_EPI_BIAS (flags 0x%x)",
                                        flags);
  if (w_dtype == WE_INT4) return fail(ctx, WE_EUNSUPPORTED, "int4 weights have no fused q/k epilogue");
  if ((uint64_t)(q_heads + k_heads) * 128 > p->n)
    return fail(ctx, WE_EINVAL, "q and k heads (%u + %u of 128) exceed the %u output columns", q_heads, k_heads, p->n);
  if ((cos_t == nullptr) != (sin_t == nullptr)) return fail(ctx, WE_EINVAL, "cos and sin go together");
  int rc = check_span(ctx, norm_q, q_heads ? 128 * 4 : 0, "norm_q");
  if (!rc) rc = check_span(ctx, norm_k, k_heads ? 128 * 4 : 0, "norm_k");
  const uint64_t rot = cos_t && p->m > rope_from ? (uint64_t)(p->m - rope_from) * 64 * 4 : 0;
  if (!rc) rc = check_span(ctx, cos_t, rot, "cos");
  if (!rc) rc = check_span(ctx, sin_t, rot, "sin");
  if (rc) return rc;
  const QkFuse qk{q_heads, k_heads, eps, offset, norm_q, norm_k, rope_from, cos_t, sin_t};
  return matmul_impl(ctx, p, x_dtype, x, w_dtype, w, nullptr, 0, y_dtype, y, bias, flags, nullptr, nullptr, false, 0,
                     &qk);
}

namespace {
// The checks every matmul entry point makes: the 3x3 convolution input's parameters, multiples of 4, dtypes,
// flags, and the extents of x, y, bias, gate and the residual / aux operand, so that no launch can read or write
// outside its buffers. Sets the split-K slice count and slice length; *empty when M or N is 0 (nothing to launch).
int check_gemm(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, int y_dtype,
               const void* y, const float* bias, uint32_t flags, const float* gate, const void* res, int mul,
               const QkFuse* qk, uint32_t* splits_out, uint32_t* kc_out, bool* empty) {
  *empty = true;
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!p) return fail(ctx, WE_EINVAL, "params is null");
  const bool conv = p->width || p->cin;
  if (conv) {
    // the 3x3 convolution input (src/kernels/matmul.ts:74-83, conv3x3Params :268-272)
    if (!p->width || !p->cin || p->cin % 4) return fail(ctx, WE_EINVAL, "cin must be a multiple of 4, got %u", p->cin);
    if (p->k != 9 * p->cin) return fail(ctx, WE_EINVAL, "a 3x3 convolution has K = 9 * cin (K %u, cin %u)", p->k, p->cin);
    if (p->m % p->width) return fail(ctx, WE_EINVAL, "M (%u pixels) is not a whole number of rows of width %u", p->m,
                                    p->width);
    if (w_dtype == WE_INT4) return fail(ctx, WE_EUNSUPPORTED, "int4 weights have no 3x3 convolution input");
    if (gate || res || mul || qk) return fail(ctx, WE_EUNSUPPORTED, "the 3x3 convolution input takes plain epilogues");
    if ((uintptr_t)x % 16) return fail(ctx, WE_EINVAL, "the convolution's image must be 16-byte aligned");
  }
  {
    const char* names[5] = {"K", "xStride", "wStride", "xOffset", "wOffset"};
    const uint32_t vals[5] = {p->k, p->x_stride, p->w_stride, p->x_offset, p->w_offset};
    for (int i = 0; i < 5; i++)
      if (vals[i] % 4) return fail(ctx, WE_EINVAL, "%s must be a multiple of 4, got %u", names[i], vals[i]);
  }
  if (!is_act(x_dtype)) return fail(ctx, WE_EINVAL, "x dtype %d is not f32 / f16 / bf16", x_dtype);
  if (!is_act(y_dtype)) return fail(ctx, WE_EINVAL, "y dtype %d is not f32 / f16 / bf16", y_dtype);
  if (!(is_act(w_dtype) || w_dtype == WE_FP8_E4M3 || w_dtype == WE_INT4))
    return fail(ctx, WE_EINVAL, "weight dtype %d is not fp8 / bf16 / f16 / f32 / int4", w_dtype);
  if (flags & ~(WE_EPI_ACCUMULATE | WE_EPI_SPLIT_K | WE_EPI_BIAS | WE_EPI_GELU_TANH))
    return fail(ctx, WE_EINVAL, "unknown epilogue flags 0x%x", flags);
  const bool split = (flags & WE_EPI_SPLIT_K) != 0;
  const uint32_t splits = split ? (p->k_split < 1 ? 1 : p->k_split) : 1;
  *empty = p->m == 0 || p->n == 0;
  if (*empty) return WE_OK;
  const uint32_t kc = split ? ((p->k + splits - 1) / splits + 15) / 16 * 16 : p->k;

  // extents of every operand (in bytes), so that no launch can read or write outside its buffers
  const uint64_t xb = elem_bytes(x_dtype), yb = elem_bytes(y_dtype);
  const uint64_t x_need = conv ? (uint64_t)p->m * p->cin * xb
                               : p->k ? ((uint64_t)p->x_offset + (uint64_t)(p->m - 1) * p->x_stride + p->k) * xb : 0;
  const uint64_t y_rows = (uint64_t)p->m * splits;
  const uint64_t y_need = ((uint64_t)p->y_offset + (y_rows - 1) * p->y_stride + p->n) * yb;
  int rc = check_span(ctx, x, x_need, "x");
  if (!rc) rc = check_span(ctx, y, y_need, "y");
  if (!rc && (flags & WE_EPI_BIAS)) rc = check_span(ctx, bias, (uint64_t)p->n * 4, "bias");
  if (!rc && gate) rc = check_span(ctx, gate, (uint64_t)p->n * 4, "gate");
  if (!rc && res) rc = check_span(ctx, res, y_need, mul ? "aux" : "residual");
  if (rc) return rc;
  *splits_out = splits;
  *kc_out = kc;
  return WE_OK;
}

// The GemmLaunch of a checked matmul with 16-bit / fp8 / f32 weights: operands, shape, epilogue, and the context's
// kernel-choice switches (tile configuration, general kernel, reduce mapping) of sweeps and tests.
void fill_gemm(we::GemmLaunch& L, const we::Tuning& t, const we_matmul_params* p, int x_dtype, const void* x,
               int w_dtype, const void* w, int y_dtype, void* y, const float* bias, uint32_t flags, const float* gate,
               const void* res, int mul, uint32_t splits, uint32_t kc) {
  const bool conv = p->width || p->cin;
  L = we::GemmLaunch{};
  L.x = x;
  L.w = w;
  L.y = y;
  L.bias = bias;
  L.gate = gate;
  L.res = res;
  L.mul = mul;
  L.conv_width = conv ? p->width : 0;
  L.conv_cin = conv ? p->cin : 0;
  L.x_dtype = x_dtype;
  L.w_dtype = w_dtype;
  L.y_dtype = y_dtype;
  L.m = p->m;
  L.n = p->n;
  L.k = p->k;
  L.scale = p->scale;
  L.x_stride = p->x_stride;
  L.w_stride = p->w_stride;
  L.y_stride = p->y_stride;
  L.x_offset = p->x_offset;
  L.w_offset = p->w_offset;
  L.y_offset = p->y_offset;
  L.splits = splits;
  L.kc = kc;
  L.flags = flags;
  L.cfg = t.gemm_cfg;
  L.generic = t.gemm_generic;
  L.reduce_xcd = t.gemm_reduce_xcd;
  L.rsplits = 1;
  L.rcfg = -1;
  L.rkc = L.k;
  L.scratch = nullptr;
}

int matmul_impl(we_ctx* ctx, const we_matmul_params* p, int x_dtype, const void* x, int w_dtype, const void* w,
                const void* w_scales, uint32_t group, int y_dtype, void* y, const float* bias, uint32_t flags,
                const float* gate, const void* res, bool noalloc, int mul, const QkFuse* qk) {
  uint32_t splits = 1, kc = 0;
  bool empty = true;
  int rc = check_gemm(ctx, p, x_dtype, x, w_dtype, y_dtype, y, bias, flags, gate, res, mul, qk, &splits, &kc, &empty);
  if (rc || empty) return rc;
  const bool split = (flags & WE_EPI_SPLIT_K) != 0;
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");

  if (w_dtype == WE_INT4) {
    if (split) return fail(ctx, WE_EUNSUPPORTED, "int4 weights have no split-K mode (the kernel splits K itself)");
    if (group == 0 || group % 64 || p->k % group)
      return fail(ctx, WE_EUNSUPPORTED, "int4 needs a group size that is a multiple of 64 and divides K (group %u, K %u)",
                  group, p->k);
    if (p->w_stride != p->k || p->w_offset != 0)
      return fail(ctx, WE_EUNSUPPORTED, "int4 weights must be contiguous [N, K/8] words (wStride = K, wOffset = 0)");
    const uint32_t align = x_dtype == WE_F32 ? 4 : 8;
    if (p->x_stride % align || p->x_offset % align || ((uintptr_t)x % 16))
      return fail(ctx, WE_EUNSUPPORTED, "int4 path needs 16-byte aligned x rows (xStride and xOffset multiples of %u)",
                  align);
    rc = check_span(ctx, w, (uint64_t)p->n * p->k / 2, "w");
    if (!rc) rc = check_span(ctx, w_scales, (uint64_t)p->n * (p->k / group) * 2, "w_scales");
    if (rc) return rc;
    we::Int4Launch L{};
    L.x = x;
    L.w = (const uint32_t*)w;
    L.scales = (const uint16_t*)w_scales;
    L.y = y;
    L.bias = bias;
    L.gate = gate;
    L.res = res;
    L.x_dtype = x_dtype;
    L.y_dtype = y_dtype;
    L.m = p->m;
    L.n = p->n;
    L.k = p->k;
    L.group = group;
    L.scale = p->scale;
    L.x_stride = p->x_stride;
    L.y_stride = p->y_stride;
    L.x_offset = p->x_offset;
    L.y_offset = p->y_offset;
    L.flags = flags;
    L.path = ctx->tune.int4_path;
    hipError_t e = we::int4_launch(L, ctx->compute);
    if (e != hipSuccess) return hip_fail(ctx, e, "int4 launch");
    return WE_OK;
  }

  const uint64_t wb = elem_bytes(w_dtype);
  const uint64_t w_need = p->k ? ((uint64_t)p->w_offset + (uint64_t)(p->n - 1) * p->w_stride + p->k) * wb : 0;
  rc = check_span(ctx, w, w_need, "w");
  if (rc) return rc;
  we::GemmLaunch L;
  fill_gemm(L, ctx->tune, p, x_dtype, x, w_dtype, w, y_dtype, y, bias, flags, gate, res, mul, splits, kc);
  // f32 activations (the reference's own dtype) on the fast path: x is split once into three exact bf16 planes along K
  // in scratch ([M, 3K]: hi | mid | lo, summing to x exactly) and the fast kernel runs one GEMM over 3K with the
  // weights read at k mod K, so each product keeps all 24 bits of x. Taken when the fast kernel accepts the planes
  // (fp8 or bf16 weights, K a multiple of 64, aligned rows); otherwise, for the allocation-free entry point and for
  // split-K partial modes, the general kernel splits x into the same planes tile by tile.
  size_t plane_bytes = 0;
  if (x_dtype == WE_F32 && !noalloc && !split && !L.generic && !L.conv_width && p->k % 64 == 0 &&
      (w_dtype == WE_FP8_E4M3 || w_dtype == WE_BF16) && (uintptr_t)x % 16 == 0 &&
      (uint64_t)p->m * p->k * 3 <= (1ull << 30)) {
    we::GemmLaunch P = L;
    P.x = (const void*)(uintptr_t)256;  // placeholder with the scratch's alignment, for the check
    P.x_dtype = WE_BF16;
    P.k = 3 * p->k;
    P.kc = P.k;
    P.k_wrap = p->k;
    P.x_stride = 3 * p->k;
    P.x_offset = 0;
    if (we::gemm_fast_supported(P)) {
      L = P;
      plane_bytes = ((uint64_t)p->m * 3 * p->k * 2 + 255) / 256 * 256;
    }
  }
  bool qk_fused = false;
  if (qk && qk->q_heads + qk->k_heads) {
    L.qk_cols = (qk->q_heads + qk->k_heads) * 128;
    L.q_cols = qk->q_heads * 128;
    L.qk_rope_from = qk->rope_from;
    L.qk_eps = qk->eps;
    L.qk_offset = qk->offset;
    L.qk_norm_q = qk->norm_q;
    L.qk_norm_k = qk->norm_k;
    L.qk_cos = qk->cos_t;
    L.qk_sin = qk->sin_t;
    qk_fused = we::gemm_qk_fusable(L);
    if (!qk_fused) L.qk_cols = L.q_cols = 0;  // the plain GEMM, then the q/k pass below
  }
  we::GemmReducePlan rp{1, L.k, 0, -1};
  if (ctx->tune.gemm_splitk != 0) {  // 0: split-K off; n > 0: n slices (sweeps)
    const uint32_t force = ctx->tune.gemm_splitk > 0 ? (uint32_t)ctx->tune.gemm_splitk : 0u;
    rp = we::gemm_reduce_plan(L, force);
  }
  if (plane_bytes) {
    // scratch: the planes of x, then the split-K partial sums (if any)
    const int rc = ensure_scratch(ctx, plane_bytes + (rp.rsplits > 1 ? rp.scratch_bytes : 0));
    if (rc) return rc;
    L.x = ctx->scratch;
    const hipError_t e = we::launch_split_f32_planes((const float*)x + p->x_offset, p->m, p->k, p->x_stride,
                                                     (uint16_t*)ctx->scratch, ctx->compute);
    if (e != hipSuccess) return hip_fail(ctx, e, "f32 plane split launch");
    if (rp.rsplits > 1) {
      L.scratch = (char*)ctx->scratch + plane_bytes;
      L.rsplits = rp.rsplits;
      L.rkc = rp.rkc;
      L.rcfg = rp.rcfg;
    }
  } else {
    if (rp.rsplits > 1) {
      if (noalloc) {
        // the device's fixed scratch array: no allocation, a hard size limit
        if (rp.scratch_bytes > we::kNoallocScratchBytes)
          return fail(ctx, WE_EINVAL,
                      "this GEMM (M %u, N %u, K %u) needs %zu bytes of split-K scratch; the allocation-free entry "
                      "point has %zu (use we_matmul)",
                      p->m, p->n, p->k, rp.scratch_bytes, we::kNoallocScratchBytes);
        L.scratch = we::noalloc_scratch(ctx->device);
        if (!L.scratch) return fail(ctx, WE_EHIP, "allocation-free scratch of device %d is not set up", ctx->device);
      } else {
        const int rc = ensure_scratch(ctx, rp.scratch_bytes);
        if (rc) return rc;
        L.scratch = ctx->scratch;
      }
      L.rsplits = rp.rsplits;
      L.rkc = rp.rkc;
      L.rcfg = rp.rcfg;
    }
  }
  hipError_t e = we::gemm_launch(L, ctx->compute);
  if (e != hipSuccess) return hip_fail(ctx, e, "gemm launch");
  if (qk && !qk_fused) {
    // no head-aligned tile for this shape: the q and k heads in a pass of their own, in place
    const uint64_t yb = elem_bytes(y_dtype);
    char* base = (char*)y + (uint64_t)p->y_offset * yb;
    for (int part = 0; part < 2; part++) {
      const uint32_t heads = part ? qk->k_heads : qk->q_heads;
      if (!heads) continue;
      char* hp = base + (uint64_t)(part ? qk->q_heads * 128 : 0) * yb;
      e = we::launch_qk_norm_rope(p->m, heads, 128, qk->eps, qk->offset, part ? qk->norm_k : qk->norm_q,
                                  qk->cos_t ? qk->rope_from : p->m, 0, qk->cos_t, qk->sin_t, y_dtype, hp, p->y_stride,
                                  hp, p->y_stride, ctx->compute);
      if (e != hipSuccess) return hip_fail(ctx, e, "qk norm rope launch");
    }
  }
  return WE_OK;
}
}  // namespace

int we_matmul_group(we_ctx* ctx, uint32_t count, const we_matmul_item* items, int x_dtype, int w_dtype, int y_dtype,
                    uint32_t flags) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (count < 1 || count > 2) return fail(ctx, WE_EINVAL, "a matmul group holds 1 or 2 GEMMs, got %u", count);
  if (!items) return fail(ctx, WE_EINVAL, "items is null");
  // every item as we_matmul_gated would check it, before anything is launched
  we::GemmLaunch L[2];
  bool empty[2] = {true, true};
  for (uint32_t i = 0; i < count; i++) {
    const we_matmul_item& it = items[i];
    if (it.gate && (flags & WE_EPI_SPLIT_K))
      return fail(ctx, WE_EINVAL, "a gated residual does not combine with split-K partials");
    if (it.residual && !it.gate) return fail(ctx, WE_EINVAL, "item %u: a residual needs a gate", i);
    if (it.residual && (flags & WE_EPI_ACCUMULATE))
      return fail(ctx, WE_EINVAL, "a residual replaces accumulate: pass y as the residual to add to y");
    uint32_t splits = 1, kc = 0;
    int rc = check_gemm(ctx, it.p, x_dtype, it.x, w_dtype, y_dtype, it.y, it.bias, flags, it.gate, it.residual, 0,
                        nullptr, &splits, &kc, &empty[i]);
    if (rc) return rc;
    if (empty[i] || w_dtype == WE_INT4) continue;
    const uint64_t wb = elem_bytes(w_dtype);
    const we_matmul_params* p = it.p;
    const uint64_t w_need = p->k ? ((uint64_t)p->w_offset + (uint64_t)(p->n - 1) * p->w_stride + p->k) * wb : 0;
    rc = check_span(ctx, it.w, w_need, "w");
    if (rc) return rc;
    fill_gemm(L[i], ctx->tune, p, x_dtype, it.x, w_dtype, it.w, y_dtype, it.y, it.bias, flags, it.gate, it.residual, 0,
              splits,
              kc);
  }
  // The paired launch runs the tiles of both GEMMs at once, so it is taken only for independent items: neither item's
  // output bytes may overlap the other's output or any operand it reads (x, w, bias, gate, residual). A dependent
  // pair runs as two calls in order, item 0 first.
  auto independent = [&]() {
    struct Span {
      uintptr_t lo, hi;
    };
    // the bytes from the first element an operand's rows touch to the last (offset, rows - 1 strides, one row)
    auto rows_span = [](const void* p, uint64_t off, uint64_t rows, uint64_t stride, uint64_t cols, uint64_t eb) {
      if (!p || !rows || !cols) return Span{0, 0};
      return Span{(uintptr_t)p + (uintptr_t)(off * eb), (uintptr_t)p + (uintptr_t)((off + (rows - 1) * stride + cols) * eb)};
    };
    auto hit = [](Span a, Span b) { return a.lo < a.hi && b.lo < b.hi && a.lo < b.hi && b.lo < a.hi; };
    const uint64_t xb = elem_bytes(x_dtype), wb = elem_bytes(w_dtype), yb = elem_bytes(y_dtype);
    Span out[2], in[2][5];
    for (int i = 0; i < 2; i++) {
      const we_matmul_params* p = items[i].p;
      out[i] = rows_span(items[i].y, p->y_offset, p->m, p->y_stride, p->n, yb);
      in[i][0] = rows_span(items[i].x, p->x_offset, p->m, p->x_stride, p->k, xb);
      in[i][1] = rows_span(items[i].w, p->w_offset, p->n, p->w_stride, p->k, wb);
      in[i][2] = rows_span((flags & WE_EPI_BIAS) ? items[i].bias : nullptr, 0, 1, 0, p->n, 4);
      in[i][3] = rows_span(items[i].gate, 0, 1, 0, p->n, 4);
      in[i][4] = rows_span(items[i].residual, p->y_offset, p->m, p->y_stride, p->n, yb);  // read where y is written
    }
    if (hit(out[0], out[1])) return false;
    for (int i = 0; i < 2; i++)
      for (const Span& r : in[1 - i])
        if (hit(out[i], r)) return false;
    return true;
  };
  if (count == 2 && !empty[0] && !empty[1] && w_dtype != WE_INT4 && we::gemm_pair_ok(L[0], L[1]) && independent()) {
    HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
    const hipError_t e = we::gemm_fast_launch_pair(L[0], L[1], ctx->compute);
    return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "gemm pair launch");
  }
  for (uint32_t i = 0; i < count; i++) {
    const we_matmul_item& it = items[i];
    const int rc = matmul_impl(ctx, it.p, x_dtype, it.x, w_dtype, it.w, nullptr, 0, y_dtype, it.y, it.bias, flags,
                               it.gate, it.residual);
    if (rc) return rc;
  }
  return WE_OK;
}

// ------------------------------------------------------------------------------------------ peak probes

int we_peak(we_ctx* ctx, int kind, uint32_t workgroups, uint32_t iters, uint32_t* out, double* ops) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (kind < WE_PEAK_F32 || kind > WE_PEAK_MFMA_BF16_DATA) return fail(ctx, WE_EINVAL, "unknown peak kind %d", kind);
  if (workgroups == 0 || workgroups > (1u << 24)) return fail(ctx, WE_EINVAL, "workgroups must be in [1, 2^24], got %u", workgroups);
  const bool mfma = kind == WE_PEAK_MFMA_BF16 || kind == WE_PEAK_MFMA_BF16_DATA;
  const uint64_t threads = (uint64_t)workgroups * (mfma ? 256 : 64);
  int rc = check_span(ctx, out, threads * 4, "out");
  if (rc) return rc;
  if (ops) *ops = (double)threads * iters * (mfma ? 4096.0 : 64.0);
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  hipError_t e = we::peak_launch(kind, workgroups, iters, out, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "peak launch");
}

int we_read_peak(we_ctx* ctx, const void* buf, size_t bytes, uint32_t* out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (bytes % 16 || (uintptr_t)buf % 16) return fail(ctx, WE_EINVAL, "the read needs 16-byte aligned whole chunks");
  int rc = check_span(ctx, buf, bytes, "buf");
  if (bytes >= (1ull << 44)) return fail(ctx, WE_EINVAL, "the read is limited to 16 TB");
  if (!rc) rc = check_span(ctx, out, we::read_peak_out_words(bytes) * 4, "out");
  if (rc) return rc;
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  hipError_t e = we::read_peak_launch(buf, bytes, out, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "read peak launch");
}

// ------------------------------------------------------------------------------------------ norms, rope, elementwise

int we_rmsnorm_mod(we_ctx* ctx, uint32_t rows, uint32_t d, float eps, float offset, int dtype, const void* x,
                   const float* weight, const float* tvec, const float* table, uint32_t mod_n, float* mod, void* out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!is_act(dtype)) return fail(ctx, WE_EINVAL, "rmsnorm dtype %d is not f32 / f16 / bf16", dtype);
  if (rows == 0 || d == 0) return fail(ctx, WE_EINVAL, "rows and d must be positive (rows %u, d %u)", rows, d);
  if (mod_n < 2 * d) return fail(ctx, WE_EINVAL, "mod_n %u is less than 2 d = %u (scale and shift)", mod_n, 2 * d);
  const uint64_t n = (uint64_t)rows * d * elem_bytes(dtype), mb = (uint64_t)mod_n * 4;
  int rc = check_span(ctx, x, n, "x");
  if (!rc) rc = check_span(ctx, out, n, "out");
  if (!rc) rc = check_span(ctx, weight, (uint64_t)d * 4, "weight");
  if (!rc) rc = check_span(ctx, tvec, mb, "tvec");
  if (!rc) rc = check_span(ctx, table, mb, "table");
  if (!rc) rc = check_span(ctx, mod, mb, "mod");
  if (rc) return rc;
  // mod is written while other threads read tvec / table / x: it may not overlap any of them
  auto overlap = [](const void* a, uint64_t na, const void* b, uint64_t nb) {
    return (const char*)a < (const char*)b + nb && (const char*)b < (const char*)a + na;
  };
  if (overlap(mod, mb, tvec, mb) || overlap(mod, mb, table, mb) || overlap(mod, mb, x, n) || overlap(mod, mb, out, n))
    return fail(ctx, WE_EINVAL, "mod may not overlap tvec, table, x or out");
  HIP_OK(ctx, hipSetDevice(ctx->device), "hipSetDevice");
  hipError_t e = we::launch_rmsnorm_mod(rows, d, eps, offset, dtype, x, weight, tvec, table, mod_n, mod, out,
                                        ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "rmsnorm launch");
}

int we_rmsnorm(we_ctx* ctx, uint32_t rows, uint32_t d, float eps, float offset, int dtype, const void* x,
               const float* weight, const float* scale, const float* shift, void* out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!is_act(dtype)) return fail(ctx, WE_EINVAL, "rmsnorm dtype %d is not f32 / f16 / bf16", dtype);
  const uint64_t n = (uint64_t)rows * d * elem_bytes(dtype);
  int rc = check_span(ctx, x, n, "x");
  if (!rc) rc = check_span(ctx, out, n, "out");
  if (!rc) rc = check_span(ctx, weight, (uint64_t)d * 4, "weight");
  if (!rc && scale) rc = check_span(ctx, scale, (uint64_t)d * 4, "scale");
  if (!rc && shift) rc = check_span(ctx, shift, (uint64_t)d * 4, "shift");
  if (rc) return rc;
  hipError_t e = we::launch_rmsnorm(rows, d, eps, offset, dtype, x, weight, scale, shift, out, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "rmsnorm launch");
}

int we_rope(we_ctx* ctx, uint32_t tokens, uint32_t heads, uint32_t pairs, int half, int dtype, const void* x,
            const float* cos_t, const float* sin_t, void* out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!is_act(dtype)) return fail(ctx, WE_EINVAL, "rope dtype %d is not f32 / f16 / bf16", dtype);
  const uint64_t n = (uint64_t)tokens * heads * pairs * 2 * elem_bytes(dtype);
  int rc = check_span(ctx, x, n, "x");
  if (!rc) rc = check_span(ctx, out, n, "out");
  if (!rc) rc = check_span(ctx, cos_t, (uint64_t)tokens * pairs * 4, "cos");
  if (!rc) rc = check_span(ctx, sin_t, (uint64_t)tokens * pairs * 4, "sin");
  if (rc) return rc;
  hipError_t e = we::launch_rope(tokens, heads, pairs, half ? 1 : 0, dtype, x, cos_t, sin_t, out, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "rope launch");
}

int we_qk_norm_rope(we_ctx* ctx, uint32_t tokens, uint32_t heads, uint32_t head_dim, float eps, float offset,
                    const float* weight, uint32_t rope_from, int half, const float* cos_t, const float* sin_t,
                    int dtype, const void* x, uint32_t x_stride, void* out, uint32_t out_stride) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!is_act(dtype)) return fail(ctx, WE_EINVAL, "dtype %d is not f32 / f16 / bf16", dtype);
  if (head_dim % 2 || head_dim == 0 || head_dim > 512)
    return fail(ctx, WE_EINVAL, "head_dim must be even and at most 512, got %u", head_dim);
  const uint64_t row = (uint64_t)heads * head_dim;
  const uint64_t xs = x_stride ? x_stride : row, os = out_stride ? out_stride : row;
  if (xs < row || os < row) return fail(ctx, WE_EINVAL, "token stride below heads * head_dim (%llu)", (unsigned long long)row);
  const uint64_t esz = elem_bytes(dtype);
  const uint64_t rot_tokens = tokens > rope_from ? tokens - rope_from : 0;
  int rc = tokens ? check_span(ctx, x, ((tokens - 1) * xs + row) * esz, "x") : WE_OK;
  if (!rc && tokens) rc = check_span(ctx, out, ((tokens - 1) * os + row) * esz, "out");
  if (!rc) rc = check_span(ctx, weight, (uint64_t)head_dim * 4, "weight");
  if (!rc) rc = check_span(ctx, cos_t, rot_tokens * (head_dim / 2) * 4, "cos");
  if (!rc) rc = check_span(ctx, sin_t, rot_tokens * (head_dim / 2) * 4, "sin");
  if (rc) return rc;
  hipError_t e = we::launch_qk_norm_rope(tokens, heads, head_dim, eps, offset, weight, rope_from, half ? 1 : 0, cos_t,
                                         sin_t, dtype, x, (uint32_t)xs, out, (uint32_t)os, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "qk norm rope launch");
}

int we_attention(we_ctx* ctx, uint32_t tokens, uint32_t heads, uint32_t kv_heads, uint32_t dim, int causal, int dtype,
                 const void* q, uint32_t q_stride, const void* k, uint32_t k_stride, const void* v, uint32_t v_stride,
                 void* out, uint32_t out_stride) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (kv_heads == 0 || heads % kv_heads) return fail(ctx, WE_EINVAL, "heads must be a multiple of kvHeads");
  if (!is_act(dtype)) return fail(ctx, WE_EINVAL, "attention dtype %d is not f32 / f16 / bf16", dtype);
  const uint32_t align = dtype == WE_F32 ? 4 : 8;
  if (dim == 0 || dim % align || dim > 128)
    return fail(ctx, WE_EUNSUPPORTED, "attention dim must be a multiple of %u and at most 128, got %u", align, dim);
  const uint64_t qrow = (uint64_t)heads * dim, kvrow = (uint64_t)kv_heads * dim;
  const uint64_t qs = q_stride ? q_stride : qrow, ks = k_stride ? k_stride : kvrow;
  const uint64_t vs = v_stride ? v_stride : kvrow, os = out_stride ? out_stride : qrow;
  if (qs < qrow || os < qrow || ks < kvrow || vs < kvrow)
    return fail(ctx, WE_EINVAL, "attention token stride below the heads it holds");
  if (qs % align || ks % align || vs % align || os % align)
    return fail(ctx, WE_EINVAL, "attention token strides must be multiples of %u", align);
  if (qs > 0xffffffffull || os > 0xffffffffull) return fail(ctx, WE_EINVAL, "attention stride too large");
  const uint64_t esz = elem_bytes(dtype);
  const void* ptrs[4] = {q, k, v, out};
  for (const void* p : ptrs)
    if (((uintptr_t)p) % 16) return fail(ctx, WE_EINVAL, "attention operands must be 16-byte aligned");
  if (tokens && heads) {
    const uint64_t last = tokens - 1;
    int rc = check_span(ctx, q, (last * qs + qrow) * esz, "q");
    if (!rc) rc = check_span(ctx, k, (last * ks + kvrow) * esz, "k");
    if (!rc) rc = check_span(ctx, v, (last * vs + kvrow) * esz, "v");
    if (!rc) rc = check_span(ctx, out, (last * os + qrow) * esz, "out");
    if (rc) return rc;
  }
  we::AttnLaunch L{q, k, v, out, dtype, tokens, heads, kv_heads, dim, (uint32_t)qs, (uint32_t)ks, (uint32_t)vs,
                   (uint32_t)os, causal ? 1 : 0, ctx->tune.attn_path, nullptr};
  const size_t need = we::attention_scratch_bytes(L);
  if (need) {
    const int rc = ensure_scratch(ctx, need);
    if (rc) return rc;
    L.scratch = ctx->scratch;
  }
  hipError_t e = we::attention_launch(L, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "attention launch");
}

int we_elementwise(we_ctx* ctx, int op, size_t n, size_t d, int dtype, const void* a, const void* b, const void* c,
                   void* out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (!is_act(dtype)) return fail(ctx, WE_EINVAL, "elementwise dtype %d is not f32 / f16 / bf16", dtype);
  if (op < WE_OP_SWIGLU || op > WE_OP_SILU) return fail(ctx, WE_EINVAL, "unknown elementwise op %d", op);
  const uint64_t bytes = (uint64_t)n * elem_bytes(dtype);
  if ((op == WE_OP_GATED_ADD || op == WE_OP_ADD_BIAS) && d == 0) return fail(ctx, WE_EINVAL, "d must be positive");
  int rc = check_span(ctx, a, bytes, "a");
  if (!rc) rc = check_span(ctx, out, bytes, "out");
  if (!rc) {
    if (op == WE_OP_ADD_BIAS) rc = check_span(ctx, b, (uint64_t)(n < d ? n : d) * 4, "bias");
    else if (op != WE_OP_GELU_TANH && op != WE_OP_SILU) rc = check_span(ctx, b, bytes, "b");
  }
  if (!rc && op == WE_OP_GATED_ADD) rc = check_span(ctx, c, (uint64_t)(n < d ? n : d) * 4, "gate");
  if (rc) return rc;
  hipError_t e = we::launch_elementwise(op, n, d ? d : 1, dtype, a, b, c, out, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "elementwise launch");
}

int we_layer_sum(we_ctx* ctx, uint32_t tokens, uint32_t layers, uint32_t dim, const float* x, const float* w,
                 float* out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  int rc = check_span(ctx, x, (uint64_t)tokens * layers * dim * 4, "x");
  if (!rc) rc = check_span(ctx, w, (uint64_t)layers * 4, "w");
  if (!rc) rc = check_span(ctx, out, (uint64_t)tokens * dim * 4, "out");
  if (rc) return rc;
  hipError_t e = we::launch_layer_sum(tokens, layers, dim, x, w, out, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "layer sum launch");
}

int we_unpack_fp8(we_ctx* ctx, const void* packed, size_t n, const float* scale, float* out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  int rc = check_span(ctx, packed, n, "packed");
  if (!rc) rc = check_span(ctx, scale, 4, "scale");
  if (!rc) rc = check_span(ctx, out, (uint64_t)n * 4, "out");
  if (rc) return rc;
  hipError_t e = we::launch_unpack_fp8(packed, n, scale, out, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "unpack launch");
}

int we_dequant_int4(we_ctx* ctx, const uint32_t* words, const uint16_t* scales, uint32_t rows, uint32_t k,
                    uint32_t group, float* out) {
  if (!ctx) return fail(ctx, WE_EINVAL, "context is null");
  if (k % 8 || group == 0 || k % group) return fail(ctx, WE_EINVAL, "K must be a multiple of 8 and of the group size");
  int rc = check_span(ctx, words, (uint64_t)rows * k / 2, "words");
  if (!rc) rc = check_span(ctx, scales, (uint64_t)rows * (k / group) * 2, "scales");
  if (!rc) rc = check_span(ctx, out, (uint64_t)rows * k * 4, "out");
  if (rc) return rc;
  hipError_t e = we::launch_dequant_int4(words, scales, rows, k, group, out, ctx->compute);
  return e == hipSuccess ? WE_OK : hip_fail(ctx, e, "dequant launch");
}

}  // extern "C"
