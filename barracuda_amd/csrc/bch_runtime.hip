// bch_runtime.hip -- the C ABI of libbarracuda_hip.so (include/barracuda_hip.h).
//
// A context = one device + one HIP stream + a grow-only scratch workspace +
// a cache of loaded code objects.  This is the device half of the
// reference's GpuBackend (crates/barracuda/src/device/backend.rs:244-444):
// alloc_buffer / upload / download / dispatch, with status codes that map
// onto BarracudaError (crates/barracuda/src/error.rs:14-130).  Argument and
// shape validation happens before any HIP call so that it behaves the same
// with or without a GPU.
#include <hip/hip_runtime.h>

#include <dlfcn.h>
#include <stdarg.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include <atomic>
#include <map>
#include <mutex>
#include <set>
#include <tuple>
#include <string>
#include <unordered_map>
#include <vector>

#include "../../include/barracuda_hip.h"
#include "bch_internal.h"

// Fixed scratch of bch_sgemm_noalloc (no hipMalloc on that path): the
// skinny GEMM's split-k partials.  Each device that loads the library holds
// its own copy until the process ends.  In host code `scratch` names a
// host-side stand-in, never device memory: the device address is resolved
// once per device with hipGetSymbolAddress and only that address is used.
constexpr size_t kNoAllocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

struct bch_ctx {
  int device = -1;
  hipStream_t stream = nullptr;
  std::string last_error;
  std::string co_dir;
  std::map<std::string, hipModule_t> modules;
  void* ws = nullptr;
  size_t ws_bytes = 0;
  // Set once the context's stream has been seen under capture: a workspace
  // replaced after that may still be read by a captured graph, so it is kept
  // (in `retired`) until bch_ctx_destroy instead of being freed.
  bool seen_capture = false;
  std::vector<void*> retired;
  // Sticky: set by the first HIP error that leaves the device context
  // unusable (a kernel fault, an ECC error); every later call that would
  // touch the device fails with BCH_E_DEVICE_LOST.  The reference flags its
  // device the same way (device/wgpu_device/submission.rs:23-71, lost.store)
  // and GpuBackend::is_lost reports it (device/backend.rs:256).
  bool lost = false;
  std::string lost_reason;
  // Host-side fault injection (BARRACUDA_HIP_INJECT_HIP_ERROR, read once at
  // bch_ctx_create): the next device call reports this HIP error as if the
  // runtime had returned it, so the error translation and the lost flag can
  // be tested without making the GPU fault.
  int inject_hip_error = 0;
  // This device's copy of `scratch` (resolved at bch_ctx_create), or null
  // with the reason in scratch_error.
  void* scratch = nullptr;
  std::string scratch_error;
  // Fault word in pinned host memory (device-visible): set by a kernel that
  // gave up a bounded wait (the skinny ring GEMM's split-k combine); read on
  // the host after every synchronisation and at every call, it marks the
  // context lost.  ring_spin: that wait's poll limit
  // (BARRACUDA_HIP_RING_SPIN, read at bch_ctx_create, forces the path in
  // tests).
  unsigned* fault_host = nullptr;
  unsigned* fault_dev = nullptr;
  unsigned ring_spin = 1u << 22;
  // Device memory handed out by bch_alloc: `live` maps each block to its
  // bucket size; bch_free parks the block in `cached` for the next bch_alloc
  // of that bucket instead of freeing it (see pool_bucket).  pool_max caps
  // the parked bytes (BARRACUDA_HIP_POOL_MAX_MB, read at bch_ctx_create).
  std::unordered_map<void*, size_t> live;
  std::map<size_t, std::vector<void*>> cached;
  size_t cached_bytes = 0;
  size_t pool_max = (size_t)8 << 30;
};

struct bch_event {
  hipEvent_t ev = nullptr;
  int device = -1;
};

namespace {

thread_local std::string t_last_error;
thread_local bch::LaunchCtl t_launch_ctl;

bch_status fail(bch_ctx* ctx, bch_status st, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  if (ctx) ctx->last_error = buf;
  t_last_error = buf;
  return st;
}

// HIP errors after which the context cannot run further work: the device
// raised an exception while executing a kernel (memory fault, trap, assert,
// watchdog), an uncorrectable ECC error, or the context is gone.  HIP keeps
// reporting them on every later call; the reference's equivalent is a wgpu
// device-lost panic.
bool context_fatal(hipError_t e) {
  switch (e) {
    case hipErrorIllegalAddress:
    case hipErrorLaunchFailure:
    case hipErrorAssert:
    case hipErrorLaunchTimeOut:
    case hipErrorECCNotCorrectable:
    case hipErrorContextIsDestroyed:
      return true;
    default:
      return false;
  }
}

bch_status from_hip(bch_ctx* ctx, hipError_t e, const char* what) {
  if (e == hipSuccess) return BCH_OK;
  if (context_fatal(e)) {
    bch_status st = fail(ctx, BCH_E_DEVICE_LOST, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
    if (ctx && !ctx->lost) {
      ctx->lost = true;
      ctx->lost_reason = ctx->last_error;
    }
    return st;
  }
  bch_status st = BCH_E_DEVICE;
  if (e == hipErrorOutOfMemory) st = BCH_E_OOM;
  else if (e == hipErrorNoDevice || e == hipErrorInvalidDevice) st = BCH_E_NO_DEVICE;
  else if (e == hipErrorInvalidImage || e == hipErrorInvalidKernelFile ||
           e == hipErrorNotFound || e == hipErrorSharedObjectInitFailed ||
           e == hipErrorNoBinaryForGpu || e == hipErrorFileNotFound)
    st = BCH_E_MODULE;
  else if (e == hipErrorLaunchOutOfResources || e == hipErrorInvalidConfiguration)
    st = BCH_E_LAUNCH;
  return fail(ctx, st, "%s: %s (%d)", what, hipGetErrorString(e), (int)e);
}

// A kernel on this context gave up a bounded wait: the context is lost.
bch_status check_fault(bch_ctx* ctx) {
  if (!ctx->fault_host || *reinterpret_cast<volatile unsigned*>(ctx->fault_host) == 0) return BCH_OK;
  bch_status st = fail(ctx, BCH_E_DEVICE_LOST,
                       "split-k combine timed out in the [out, in] skinny GEMM (a partial block never arrived; "
                       "its outputs were set to NaN)");
  if (!ctx->lost) {
    ctx->lost = true;
    ctx->lost_reason = ctx->last_error;
  }
  return st;
}

// The context's stream is being captured into a graph (or a capture on it
// was invalidated and not yet ended).
bool capturing(bch_ctx* ctx) {
  hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(ctx->stream, &cs) != hipSuccess) {
    (void)hipGetLastError();
    return false;
  }
  return cs != hipStreamCaptureStatusNone;
}

// Every call that touches the device starts here.
bch_status use(bch_ctx* ctx) {
  if (ctx->lost) return fail(ctx, BCH_E_DEVICE_LOST, "device lost: %s", ctx->lost_reason.c_str());
  if (check_fault(ctx) != BCH_OK) return BCH_E_DEVICE_LOST;
  bch::launch_ctl().fault = ctx->fault_dev;
  bch::launch_ctl().spin = ctx->ring_spin;
  if (ctx->inject_hip_error) {
    const hipError_t e = static_cast<hipError_t>(ctx->inject_hip_error);
    ctx->inject_hip_error = 0;
    return from_hip(ctx, e, "injected by BARRACUDA_HIP_INJECT_HIP_ERROR");
  }
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return from_hip(ctx, e, "hipSetDevice");
  if (capturing(ctx)) ctx->seen_capture = true;
  return BCH_OK;
}

std::string lib_dir() {
  Dl_info info;
  if (dladdr(reinterpret_cast<void*>(&bch_status_string), &info) && info.dli_fname) {
    std::string p(info.dli_fname);
    size_t s = p.rfind('/');
    if (s != std::string::npos) return p.substr(0, s);
  }
  return ".";
}

bch_status ensure_ws(bch_ctx* ctx, size_t bytes) {
  if (bytes <= ctx->ws_bytes) return BCH_OK;
  // Growing allocates, and under capture it would also record the clear into
  // the caller's graph and leave earlier captures reading freed memory.
  if (capturing(ctx))
    return fail(ctx, BCH_E_UNSUPPORTED,
                "workspace of %zu bytes needed while the context's stream is being captured (it holds %zu): "
                "size it before the capture (an eager call or bch_ctx_reserve) or use bch_sgemm_noalloc",
                bytes, ctx->ws_bytes);
  if (ctx->ws) {
    hipError_t e = hipStreamSynchronize(ctx->stream);
    if (e != hipSuccess) return from_hip(ctx, e, "hipStreamSynchronize");
    if (ctx->seen_capture)
      ctx->retired.push_back(ctx->ws);  // captured graphs may still read it
    else
      (void)hipFree(ctx->ws);
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
  }
  size_t want = bytes < ((size_t)1 << 20) ? ((size_t)1 << 20) : bytes;
  hipError_t e = hipMalloc(&ctx->ws, want);
  if (e != hipSuccess) {
    ctx->ws = nullptr;
    return from_hip(ctx, e, "workspace hipMalloc");
  }
  ctx->ws_bytes = want;
  // No kernel relies on the contents (split-k partials and softmax chunk
  // states are written before they are read); the clear only keeps a fresh
  // workspace deterministic for debugging.
  return from_hip(ctx, hipMemsetAsync(ctx->ws, 0, want, ctx->stream), "workspace clear");
}

bool fail_alloc_injected() {
  const char* v = getenv("BARRACUDA_HIP_FAIL_ALLOC");
  return v && v[0] == '1';
}

// Device address of `scratch` on the current device, resolved once per
// device (hipGetSymbolAddress with that device current) and kept.
constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices];

void resolve_scratch(bch_ctx* ctx) {
  if (ctx->device < 0 || ctx->device >= kMaxDevices) {
    ctx->scratch_error = "device ordinal beyond the scratch table";
    return;
  }
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[ctx->device]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) {
      (void)hipGetLastError();
      ctx->scratch_error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e);
      return;
    }
    g_scratch_ptr[ctx->device] = p;
  }
  ctx->scratch = g_scratch_ptr[ctx->device];
}

}  // namespace

namespace bch {
LaunchCtl& launch_ctl() { return t_launch_ctl; }
}  // namespace bch

extern "C" {

const char* bch_status_string(bch_status s) {
  switch (s) {
    case BCH_OK: return "ok";
    case BCH_E_INVALID: return "invalid argument";
    case BCH_E_SHAPE: return "shape mismatch";
    case BCH_E_NO_DEVICE: return "no device available";
    case BCH_E_OOM: return "out of device memory";
    case BCH_E_MODULE: return "code object missing or invalid";
    case BCH_E_LAUNCH: return "kernel launch failed";
    case BCH_E_DEVICE: return "device error";
    case BCH_E_UNSUPPORTED: return "unsupported operation";
    case BCH_E_DEVICE_LOST: return "device lost";
    default: return "unknown status";
  }
}

const char* bch_last_error(const bch_ctx* ctx) {
  if (ctx) return ctx->last_error.c_str();
  return t_last_error.c_str();
}

bch_status bch_device_count(int* count) {
  if (!count) return fail(nullptr, BCH_E_INVALID, "bch_device_count: count is NULL");
  *count = 0;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n <= 0) {
    (void)hipGetLastError();
    return fail(nullptr, BCH_E_NO_DEVICE, "no HIP device available (hipGetDeviceCount: %s)",
                hipGetErrorString(e));
  }
  *count = n;
  return BCH_OK;
}

bch_status bch_ctx_create(int device, const char* code_object_dir, bch_ctx** out) {
  if (!out) return fail(nullptr, BCH_E_INVALID, "bch_ctx_create: out is NULL");
  *out = nullptr;
  if (device < 0) {
    const char* env = getenv("BARRACUDA_HIP_DEVICE");
    device = env ? atoi(env) : 0;
  }
  int n = 0;
  bch_status st = bch_device_count(&n);
  if (st != BCH_OK) return st;
  if (device >= n)
    return fail(nullptr, BCH_E_NO_DEVICE, "bch_ctx_create: device %d not present (%d visible)", device, n);
  bch_ctx* ctx = new bch_ctx();
  ctx->device = device;
  if (const char* inj = getenv("BARRACUDA_HIP_INJECT_HIP_ERROR")) ctx->inject_hip_error = atoi(inj);
  ctx->co_dir = code_object_dir ? code_object_dir : lib_dir();
  hipError_t e = hipSetDevice(device);
  if (e == hipSuccess) e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    st = from_hip(nullptr, e, "bch_ctx_create");
    delete ctx;
    return st;
  }
  resolve_scratch(ctx);
  if (const char* sp = getenv("BARRACUDA_HIP_RING_SPIN")) ctx->ring_spin = (unsigned)strtoul(sp, nullptr, 10);
  if (const char* pm = getenv("BARRACUDA_HIP_POOL_MAX_MB")) ctx->pool_max = (size_t)strtoull(pm, nullptr, 10) << 20;
  void* fh = nullptr;
  void* fd = nullptr;
  if (hipHostMalloc(&fh, 64, hipHostMallocMapped) == hipSuccess && fh) {
    *static_cast<volatile unsigned*>(fh) = 0;
    if (hipHostGetDevicePointer(&fd, fh, 0) == hipSuccess && fd) {
      ctx->fault_host = static_cast<unsigned*>(fh);
      ctx->fault_dev = static_cast<unsigned*>(fd);
    } else {
      (void)hipHostFree(fh);
    }
  }
  (void)hipGetLastError();
  *out = ctx;
  return BCH_OK;
}

bch_status bch_ctx_is_lost(const bch_ctx* ctx, int* lost) {
  if (!ctx || !lost) return fail(nullptr, BCH_E_INVALID, "bch_ctx_is_lost: NULL argument");
  *lost = ctx->lost ? 1 : 0;
  return BCH_OK;
}

bch_status bch_ctx_stream(const bch_ctx* ctx, void** stream) {
  if (!ctx || !stream) return fail(nullptr, BCH_E_INVALID, "bch_ctx_stream: NULL argument");
  *stream = ctx->stream;
  return BCH_OK;
}

bch_status bch_ctx_reserve(bch_ctx* ctx, size_t bytes) {
  if (!ctx) return fail(ctx, BCH_E_INVALID, "bch_ctx_reserve: ctx is NULL");
  if (bytes <= ctx->ws_bytes) return BCH_OK;
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  return ensure_ws(ctx, bytes);
}

bch_status bch_ctx_workspace_bytes(const bch_ctx* ctx, size_t* bytes) {
  if (!ctx || !bytes) return fail(nullptr, BCH_E_INVALID, "bch_ctx_workspace_bytes: NULL argument");
  *bytes = ctx->ws_bytes;
  return BCH_OK;
}

void bch_ctx_destroy(bch_ctx* ctx) {
  if (!ctx) return;
  (void)hipSetDevice(ctx->device);
  if (ctx->stream) (void)hipStreamSynchronize(ctx->stream);
  for (auto& kv : ctx->cached)
    for (void* p : kv.second) (void)hipFree(p);
  for (auto& kv : ctx->modules) (void)hipModuleUnload(kv.second);
  if (ctx->ws) (void)hipFree(ctx->ws);
  for (void* p : ctx->retired) (void)hipFree(p);
  if (ctx->fault_host) (void)hipHostFree(ctx->fault_host);
  if (ctx->stream) (void)hipStreamDestroy(ctx->stream);
  delete ctx;
}

// ---- device memory: freed blocks are kept per context and handed out again ----
// The reference hands each op's output from a pool of power-of-two buckets
// (device/tensor_context/pool.rs:268-334, acquire_pooled; ops/matmul.rs:128
// "zero allocation in steady state").  Here bch_free parks a block in its
// bucket and the next bch_alloc of that bucket takes it back, so a loop of
// ops on fresh outputs makes no hipMalloc and no hipFree (which waits for the
// device) after its first pass.  Reuse needs no wait: every call of a context
// runs in order on its one stream, so work queued after bch_alloc returns a
// parked block runs after the work that still read it.  Buckets: powers of
// two from 256 bytes to 64 MiB, then multiples of 2 MiB (a large block
// wastes at most 2 MiB).  A failed hipMalloc releases the parked blocks and
// tries once more; parked bytes beyond pool_max are freed at once.
constexpr size_t kPoolMinBytes = 256;
constexpr size_t kPoolPow2Max = (size_t)64 << 20;
constexpr size_t kPoolLargeStep = (size_t)2 << 20;

static size_t pool_bucket(size_t bytes) {
  if (bytes <= kPoolMinBytes) return kPoolMinBytes;
  if (bytes <= kPoolPow2Max) {
    size_t b = kPoolMinBytes;
    while (b < bytes) b <<= 1;
    return b;
  }
  return (bytes + kPoolLargeStep - 1) / kPoolLargeStep * kPoolLargeStep;
}

// Frees every parked block (after the stream's queued work).
static hipError_t pool_release(bch_ctx* ctx) {
  if (ctx->cached_bytes == 0) return hipSuccess;
  hipError_t e = hipStreamSynchronize(ctx->stream);
  for (auto& kv : ctx->cached)
    for (void* p : kv.second) {
      const hipError_t f = hipFree(p);
      if (e == hipSuccess) e = f;
    }
  ctx->cached.clear();
  ctx->cached_bytes = 0;
  return e;
}

bch_status bch_alloc(bch_ctx* ctx, size_t bytes, void** dptr) {
  if (!ctx || !dptr) return fail(ctx, BCH_E_INVALID, "bch_alloc: NULL argument");
  *dptr = nullptr;
  if (bytes == 0) return BCH_OK;
  if (fail_alloc_injected())
    return fail(ctx, BCH_E_OOM, "bch_alloc: allocation of %zu bytes failed (injected by BARRACUDA_HIP_FAIL_ALLOC)", bytes);
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  const size_t b = pool_bucket(bytes);
  auto it = ctx->cached.find(b);
  if (it != ctx->cached.end() && !it->second.empty()) {
    *dptr = it->second.back();
    it->second.pop_back();
    ctx->cached_bytes -= b;
    ctx->live[*dptr] = b;
    return BCH_OK;
  }
  hipError_t e = hipMalloc(dptr, b);
  if (e == hipErrorOutOfMemory && ctx->cached_bytes > 0) {
    (void)hipGetLastError();
    e = pool_release(ctx);
    if (e == hipSuccess) e = hipMalloc(dptr, b);
  }
  if (e != hipSuccess) {
    *dptr = nullptr;
    (void)hipGetLastError();
    return from_hip(ctx, e, "bch_alloc");
  }
  ctx->live[*dptr] = b;
  return BCH_OK;
}

bch_status bch_free(bch_ctx* ctx, void* dptr) {
  if (!ctx) return fail(ctx, BCH_E_INVALID, "bch_free: ctx is NULL");
  if (!dptr) return BCH_OK;
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  auto it = ctx->live.find(dptr);
  if (it != ctx->live.end()) {
    const size_t b = it->second;
    ctx->live.erase(it);
    if (ctx->cached_bytes + b <= ctx->pool_max) {
      ctx->cached[b].push_back(dptr);
      ctx->cached_bytes += b;
      return BCH_OK;
    }
  }
  // Not parked (over the cap, or memory bch_alloc did not hand out): work queued
  // on this context may still read it.
  hipError_t e = hipStreamSynchronize(ctx->stream);
  if (e == hipSuccess) e = hipFree(dptr);
  return from_hip(ctx, e, "bch_free");
}

bch_status bch_upload(bch_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (bytes && (!dst || !src))) return fail(ctx, BCH_E_INVALID, "bch_upload: NULL argument");
  if (!bytes) return BCH_OK;
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);  // src may be reused at once
  return from_hip(ctx, e, "bch_upload");
}

bch_status bch_download(bch_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (bytes && (!dst || !src))) return fail(ctx, BCH_E_INVALID, "bch_download: NULL argument");
  if (!bytes) return BCH_OK;
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  hipError_t e = hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  st = from_hip(ctx, e, "bch_download");
  return st != BCH_OK ? st : check_fault(ctx);
}

bch_status bch_memset(bch_ctx* ctx, void* dst, int value, size_t bytes) {
  if (!ctx || (bytes && !dst)) return fail(ctx, BCH_E_INVALID, "bch_memset: NULL argument");
  if (!bytes) return BCH_OK;
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  return from_hip(ctx, hipMemsetAsync(dst, value, bytes, ctx->stream), "bch_memset");
}

bch_status bch_copy(bch_ctx* ctx, void* dst, const void* src, size_t bytes) {
  if (!ctx || (bytes && (!dst || !src))) return fail(ctx, BCH_E_INVALID, "bch_copy: NULL argument");
  if (!bytes) return BCH_OK;
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  return from_hip(ctx, bch::launch_copy(ctx->stream, dst, src, bytes), "bch_copy launch");
}

bch_status bch_sync(bch_ctx* ctx) {
  if (!ctx) return fail(ctx, BCH_E_INVALID, "bch_sync: ctx is NULL");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  st = from_hip(ctx, hipStreamSynchronize(ctx->stream), "bch_sync");
  return st != BCH_OK ? st : check_fault(ctx);
}

bch_status bch_sgemm_ex(bch_ctx* ctx, int transb, int m, int n, int k, const float* A, int lda, const float* B,
                        int ldb, const float* bias, int act, float* C, int ldc) {
  if (transb != 0 && transb != 1) return fail(ctx, BCH_E_INVALID, "linear: transb must be 0 or 1 (got %d)", transb);
  if (act != BCH_ACT_NONE && act != BCH_ACT_RELU && act != BCH_ACT_GELU)
    return fail(ctx, BCH_E_INVALID, "linear: unknown activation %d", act);
  if (m < 0 || n < 0 || k < 0)
    return fail(ctx, BCH_E_SHAPE, "linear: negative dimension (m=%d, n=%d, k=%d)", m, n, k);
  const int kmin = k > 1 ? k : 1, nmin = n > 1 ? n : 1;
  if (lda < kmin || ldb < (transb ? kmin : nmin) || ldc < nmin)
    return fail(ctx, BCH_E_SHAPE, "linear: leading dimension too small (lda=%d k=%d, ldb=%d %s=%d, ldc=%d n=%d)",
                lda, k, ldb, transb ? "k" : "n", transb ? k : n, ldc, n);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "linear: ctx is NULL");
  if (m == 0 || n == 0) return BCH_OK;
  if (!C || (k > 0 && (!A || !B))) return fail(ctx, BCH_E_INVALID, "linear: NULL buffer");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  size_t wsb = bch::sgemm_ex_workspace_bytes(transb != 0, 1, m, n, k, lda, ldb);
  if (wsb) {
    st = ensure_ws(ctx, wsb);
    if (st != BCH_OK) return st;
  }
  hipError_t e = bch::launch_sgemm_ex(ctx->stream, transb != 0, 1, m, n, k, A, lda, 0, B, ldb, 0, bias, act, C,
                                      ldc, 0, ctx->ws, ctx->ws_bytes);
  return from_hip(ctx, e, "linear launch");
}

bch_status bch_sgemm_strided_batched(bch_ctx* ctx, int batch, int m, int n, int k,
                                     const float* A, long long strideA, const float* B,
                                     long long strideB, float* C, long long strideC);

bch_status bch_sgemm(bch_ctx* ctx, int m, int n, int k, const float* A, int lda,
                     const float* B, int ldb, float* C, int ldc) {
  if (m < 0 || n < 0 || k < 0)
    return fail(ctx, BCH_E_SHAPE, "matmul: negative dimension (m=%d, n=%d, k=%d)", m, n, k);
  if (lda < (k > 1 ? k : 1) || ldb < (n > 1 ? n : 1) || ldc < (n > 1 ? n : 1))
    return fail(ctx, BCH_E_SHAPE, "matmul: leading dimension too small (lda=%d k=%d, ldb=%d n=%d, ldc=%d n=%d)",
                lda, k, ldb, n, ldc, n);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "matmul: ctx is NULL");
  if (m == 0 || n == 0) return BCH_OK;
  if (!C || (k > 0 && (!A || !B))) return fail(ctx, BCH_E_INVALID, "matmul: NULL buffer");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  size_t wsb = bch::sgemm_workspace_bytes(1, m, n, k);
  if (wsb) {
    st = ensure_ws(ctx, wsb);
    if (st != BCH_OK) return st;
  }
  hipError_t e = bch::launch_sgemm(ctx->stream, 1, m, n, k, A, lda, 0, B, ldb, 0, C, ldc, 0,
                                   ctx->ws, ctx->ws_bytes);
  return from_hip(ctx, e, "matmul launch");
}

bch_status bch_sgemm_noalloc(bch_ctx* ctx, int m, int n, int k, const float* A, int lda,
                             const float* B, int ldb, float* C, int ldc) {
  if (m < 0 || n < 0 || k < 0)
    return fail(ctx, BCH_E_SHAPE, "matmul: negative dimension (m=%d, n=%d, k=%d)", m, n, k);
  if (lda < (k > 1 ? k : 1) || ldb < (n > 1 ? n : 1) || ldc < (n > 1 ? n : 1))
    return fail(ctx, BCH_E_SHAPE, "matmul: leading dimension too small (lda=%d k=%d, ldb=%d n=%d, ldc=%d n=%d)",
                lda, k, ldb, n, ldc, n);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "matmul: ctx is NULL");
  if (m == 0 || n == 0) return BCH_OK;
  if (!C || (k > 0 && (!A || !B))) return fail(ctx, BCH_E_INVALID, "matmul: NULL buffer");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  // sized with this device current (the stream-K plans take one workgroup per CU); the tile
  // path's optional hybrid-plan scratch is used when it fits in the fixed scratch
  const size_t wsb = bch::sgemm_required_workspace_bytes(1, m, n, k);
  if (wsb > kNoAllocScratchBytes)
    return fail(ctx, BCH_E_UNSUPPORTED,
                "matmul (no-alloc): m=%d n=%d k=%d needs %zu bytes of scratch, more than the fixed %zu",
                m, n, k, wsb, kNoAllocScratchBytes);
  if (wsb && !ctx->scratch)
    return fail(ctx, BCH_E_DEVICE, "matmul (no-alloc): fixed scratch unavailable (%s)", ctx->scratch_error.c_str());
  hipError_t e = bch::launch_sgemm(ctx->stream, 1, m, n, k, A, lda, 0, B, ldb, 0, C, ldc, 0, ctx->scratch,
                                   ctx->scratch ? kNoAllocScratchBytes : 0);
  return from_hip(ctx, e, "matmul (no-alloc) launch");
}

bch_status bch_sgemm_strided_batched(bch_ctx* ctx, int batch, int m, int n, int k,
                                     const float* A, long long strideA, const float* B,
                                     long long strideB, float* C, long long strideC) {
  if (batch < 0 || m < 0 || n < 0 || k < 0)
    return fail(ctx, BCH_E_SHAPE, "batch_matmul: negative dimension (batch=%d, m=%d, n=%d, k=%d)", batch, m, n, k);
  if (batch > 1 && (strideA < (long long)m * k || strideB < (long long)k * n || strideC < (long long)m * n))
    return fail(ctx, BCH_E_SHAPE, "batch_matmul: batch stride smaller than one matrix (sA=%lld, sB=%lld, sC=%lld)",
                strideA, strideB, strideC);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "batch_matmul: ctx is NULL");
  if (batch == 0 || m == 0 || n == 0) return BCH_OK;
  if (!C || (k > 0 && (!A || !B))) return fail(ctx, BCH_E_INVALID, "batch_matmul: NULL buffer");
  if (batch > 65535) return fail(ctx, BCH_E_UNSUPPORTED, "batch_matmul: batch %d > 65535", batch);
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  size_t wsb = bch::sgemm_workspace_bytes(batch, m, n, k);
  if (wsb) {
    st = ensure_ws(ctx, wsb);
    if (st != BCH_OK) return st;
  }
  const int lda = k > 0 ? k : 1, ldb = n, ldc = n;
  hipError_t e = bch::launch_sgemm(ctx->stream, batch, m, n, k, A, lda, strideA, B, ldb, strideB, C,
                                   ldc, strideC, ctx->ws, ctx->ws_bytes);
  return from_hip(ctx, e, "batch_matmul launch");
}

bch_status bch_dgemm(bch_ctx* ctx, int transa, int transb, int batch, int m, int n, int k, double alpha,
                     const double* A, int lda, long long strideA, const double* B, int ldb, long long strideB,
                     double beta, double* C, int ldc, long long strideC) {
  if ((transa != 0 && transa != 1) || (transb != 0 && transb != 1))
    return fail(ctx, BCH_E_INVALID, "gemm_f64: transpose flags must be 0 or 1 (got %d, %d)", transa, transb);
  if (batch < 0 || m < 0 || n < 0 || k < 0)
    return fail(ctx, BCH_E_SHAPE, "gemm_f64: negative dimension (batch=%d, m=%d, n=%d, k=%d)", batch, m, n, k);
  const int ar = transa ? m : k, br = transb ? k : n;  // stored row lengths of A and B
  if (lda < (ar > 1 ? ar : 1) || ldb < (br > 1 ? br : 1) || ldc < (n > 1 ? n : 1))
    return fail(ctx, BCH_E_SHAPE, "gemm_f64: leading dimension too small (lda=%d needs %d, ldb=%d needs %d, "
                "ldc=%d needs %d)", lda, ar, ldb, br, ldc, n);
  // Extent of one stored matrix: (rows - 1) * ld + row length, 0 when empty
  // (k == 0 leaves A and B empty whatever lda and ldb are).
  auto extent = [](long long rows, long long cols, long long ld) {
    return rows > 0 && cols > 0 ? (rows - 1) * ld + cols : 0LL;
  };
  const long long asz = extent(transa ? k : m, ar, lda), bsz = extent(transb ? n : k, br, ldb);
  if (batch > 1 && (strideA < asz || strideB < bsz || strideC < extent(m, n, ldc)))
    return fail(ctx, BCH_E_SHAPE, "gemm_f64: batch stride smaller than one matrix (sA=%lld, sB=%lld, sC=%lld)",
                strideA, strideB, strideC);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "gemm_f64: ctx is NULL");
  if (batch == 0 || m == 0 || n == 0) return BCH_OK;
  if (!C || (k > 0 && (!A || !B))) return fail(ctx, BCH_E_INVALID, "gemm_f64: NULL buffer");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  const size_t wsb = bch::dgemm_workspace_bytes(batch, m, n, k);
  if (wsb) {
    st = ensure_ws(ctx, wsb);
    if (st != BCH_OK) return st;
  }
  return from_hip(ctx,
                  bch::launch_dgemm(ctx->stream, transa != 0, transb != 0, batch, m, n, k, alpha, A, lda, strideA,
                                    B, ldb, strideB, beta, C, ldc, strideC, ctx->ws, ctx->ws_bytes),
                  "gemm_f64 launch");
}

bch_status bch_softmax_rows(bch_ctx* ctx, long long rows, long long cols, const float* in, float* out) {
  if (rows < 1 || cols < 1)
    return fail(ctx, BCH_E_SHAPE, "softmax: empty dimension (rows=%lld, cols=%lld)", rows, cols);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "softmax: ctx is NULL");
  if (!in || !out) return fail(ctx, BCH_E_INVALID, "softmax: NULL buffer");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  size_t wsb = bch::softmax_workspace_bytes(rows, cols);
  if (wsb) {
    st = ensure_ws(ctx, wsb);
    if (st != BCH_OK) return st;
  }
  return from_hip(ctx, bch::launch_softmax_rows(ctx->stream, rows, cols, in, out, ctx->ws, ctx->ws_bytes),
                  "softmax launch");
}

bch_status bch_softmax_rows_f64(bch_ctx* ctx, long long rows, long long cols, const double* in, double* out) {
  if (rows < 1 || cols < 1)
    return fail(ctx, BCH_E_SHAPE, "softmax_f64: empty dimension (rows=%lld, cols=%lld)", rows, cols);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "softmax_f64: ctx is NULL");
  if (!in || !out) return fail(ctx, BCH_E_INVALID, "softmax_f64: NULL buffer");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  return from_hip(ctx, bch::launch_softmax_rows_f64(ctx->stream, rows, cols, in, out), "softmax_f64 launch");
}

bch_status bch_elementwise(bch_ctx* ctx, int op, long long n, const float* a, const float* b, const float* c,
                           float scalar, float* out) {
  if (op < BCH_EW_ADD || op > BCH_EW_GELU) return fail(ctx, BCH_E_INVALID, "elementwise: unknown op %d", op);
  if (n < 0) return fail(ctx, BCH_E_SHAPE, "elementwise: negative element count %lld", n);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "elementwise: ctx is NULL");
  if (n == 0) return BCH_OK;
  const bool needs_b = op == BCH_EW_ADD || op == BCH_EW_SUB || op == BCH_EW_MUL || op == BCH_EW_FMA;
  if (!a || !out || (needs_b && !b) || (op == BCH_EW_FMA && !c))
    return fail(ctx, BCH_E_INVALID, "elementwise: NULL buffer");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  return from_hip(ctx, bch::launch_elementwise(ctx->stream, op, n, a, b, c, scalar, out), "elementwise launch");
}

bch_status bch_layer_norm(bch_ctx* ctx, long long rows, long long cols, float eps, const float* in, float* out) {
  if (rows < 1 || cols < 1)
    return fail(ctx, BCH_E_SHAPE, "layer_norm: empty dimension (rows=%lld, cols=%lld)", rows, cols);
  if (!(eps >= 0.0f)) return fail(ctx, BCH_E_INVALID, "layer_norm: epsilon must be >= 0 (got %g)", (double)eps);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "layer_norm: ctx is NULL");
  if (!in || !out) return fail(ctx, BCH_E_INVALID, "layer_norm: NULL buffer");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  return from_hip(ctx, bch::launch_layer_norm(ctx->stream, rows, cols, eps, in, out), "layer_norm launch");
}

namespace {

bch_status head_permute(bch_ctx* ctx, bool concat, int B, int S, int H, int D, const float* in, float* out) {
  const char* op = concat ? "head_concat" : "head_split";
  if (B < 1 || S < 1 || H < 1 || D < 1)
    return fail(ctx, BCH_E_SHAPE, "%s: empty dimension (B=%d, S=%d, H=%d, D=%d)", op, B, S, H, D);
  if ((long long)H * D > 0x7fffffffLL || (long long)S * D > 0x7fffffffLL)
    return fail(ctx, BCH_E_UNSUPPORTED, "%s: S*D or H*D above 2^31 - 1 (S=%d, H=%d, D=%d)", op, S, H, D);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "%s: ctx is NULL", op);
  if (!in || !out) return fail(ctx, BCH_E_INVALID, "%s: NULL buffer", op);
  if (in == out) return fail(ctx, BCH_E_INVALID, "%s: in and out must be different buffers", op);
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  return from_hip(ctx, bch::launch_head_permute(ctx->stream, concat, B, S, H, D, in, out),
                  concat ? "head_concat launch" : "head_split launch");
}

}  // namespace

bch_status bch_head_split(bch_ctx* ctx, int B, int S, int H, int D, const float* in, float* out) {
  return head_permute(ctx, false, B, S, H, D, in, out);
}

bch_status bch_head_concat(bch_ctx* ctx, int B, int S, int H, int D, const float* in, float* out) {
  return head_permute(ctx, true, B, S, H, D, in, out);
}

bch_status bch_softmax_axis(bch_ctx* ctx, long long outer, long long axis, long long inner,
                            const float* in, float* out) {
  if (outer < 1 || axis < 1 || inner < 1)
    return fail(ctx, BCH_E_SHAPE, "softmax_dim: empty dimension (outer=%lld, axis=%lld, inner=%lld)", outer,
                axis, inner);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "softmax_dim: ctx is NULL");
  if (!in || !out) return fail(ctx, BCH_E_INVALID, "softmax_dim: NULL buffer");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  size_t wsb = bch::softmax_axis_workspace_bytes(outer, axis, inner);
  if (wsb) {
    st = ensure_ws(ctx, wsb);
    if (st != BCH_OK) return st;
  }
  // softmax_dim's own semantics: a slice whose sum is not > 0 stays un-normalised
  return from_hip(ctx, bch::launch_softmax_axis(ctx->stream, outer, axis, inner, in, out, ctx->ws,
                                                ctx->ws_bytes, true),
                  "softmax_dim launch");
}

namespace {

// Both attention entry points after validation: the fused kernel up to
// D = kSdpaFusedMaxD, the chunked three-step path (in the workspace) above.
bch_status sdpa_run(bch_ctx* ctx, int B, int H, int Hkv, int Sq, int Skv, int D, float scale, int causal,
                    const float* q, const float* k, const float* v, float* o, const bch::SdpaStrides& s) {
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  if (D <= bch::kSdpaFusedMaxD)
    return from_hip(ctx, bch::launch_sdpa_strided(ctx->stream, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, s),
                    "attention launch");
  if (s.q.row > 0x7fffffffLL || s.k.row > 0x7fffffffLL || s.v.row > 0x7fffffffLL || s.o.row > 0x7fffffffLL)
    return fail(ctx, BCH_E_UNSUPPORTED, "attention: head dimension %d > %d needs row strides below 2^31", D,
                bch::kSdpaFusedMaxD);
  if (Hkv > 65535)
    return fail(ctx, BCH_E_UNSUPPORTED, "attention: head dimension %d > %d needs at most 65535 key/value heads", D,
                bch::kSdpaFusedMaxD);
  st = ensure_ws(ctx, bch::sdpa_wide_workspace_bytes(Hkv, Sq, Skv, D, causal, s.q.row, s.k.row));
  if (st != BCH_OK) return st;
  return from_hip(ctx,
                  bch::launch_sdpa_wide(ctx->stream, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, s, ctx->ws,
                                        ctx->ws_bytes),
                  "attention launch");
}

}  // namespace

bch_status bch_sdpa_fwd(bch_ctx* ctx, int B, int H, int Sq, int Skv, int D, float scale, int causal,
                        const float* q, const float* k, const float* v, float* o) {
  if (B < 1 || H < 1 || Sq < 1 || Skv < 1 || D < 1)
    return fail(ctx, BCH_E_SHAPE, "attention: empty dimension (B=%d, H=%d, Sq=%d, Skv=%d, D=%d)", B, H, Sq,
                Skv, D);
  if (causal && Sq != Skv)
    return fail(ctx, BCH_E_SHAPE, "attention: causal mask needs Sq == Skv (shape mismatch %d vs %d)", Sq, Skv);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "attention: ctx is NULL");
  if (!q || !k || !v || !o) return fail(ctx, BCH_E_INVALID, "attention: NULL buffer");
  bch::SdpaStrides s;
  s.q = s.o = bch::SdpaLayout{(long long)H * Sq * D, (long long)Sq * D, D};
  s.k = s.v = bch::SdpaLayout{(long long)H * Skv * D, (long long)Skv * D, D};
  return sdpa_run(ctx, B, H, H, Sq, Skv, D, scale, causal, q, k, v, o, s);
}

bch_status bch_sdpa_fwd_ex(bch_ctx* ctx, int B, int H, int Hkv, int Sq, int Skv, int D, float scale, int causal,
                           const float* q, bch_attn_layout ql, const float* k, bch_attn_layout kl, const float* v,
                           bch_attn_layout vl, float* o, bch_attn_layout ol) {
  if (B < 1 || H < 1 || Hkv < 1 || Sq < 1 || Skv < 1 || D < 1)
    return fail(ctx, BCH_E_SHAPE, "attention: empty dimension (B=%d, H=%d, Hkv=%d, Sq=%d, Skv=%d, D=%d)", B, H,
                Hkv, Sq, Skv, D);
  if (H % Hkv != 0)
    return fail(ctx, BCH_E_INVALID, "num_q_heads (%d) must be divisible by num_kv_heads (%d)", H, Hkv);
  if (causal && Sq != Skv)
    return fail(ctx, BCH_E_SHAPE, "attention: causal mask needs Sq == Skv (shape mismatch %d vs %d)", Sq, Skv);
  const bch_attn_layout* ls[4] = {&ql, &kl, &vl, &ol};
  for (int i = 0; i < 4; ++i)
    if (ls[i]->batch_stride < 0 || ls[i]->head_stride < 0 || ls[i]->row_stride < D)
      return fail(ctx, BCH_E_INVALID,
                  "attention: %c layout (batch %lld, head %lld, row %lld) needs non-negative strides and "
                  "row stride >= D = %d",
                  "qkvo"[i], ls[i]->batch_stride, ls[i]->head_stride, ls[i]->row_stride, D);
  if (!ctx) return fail(ctx, BCH_E_INVALID, "attention: ctx is NULL");
  if (!q || !k || !v || !o) return fail(ctx, BCH_E_INVALID, "attention: NULL buffer");
  bch::SdpaStrides s;
  s.q = {ql.batch_stride, ql.head_stride, ql.row_stride};
  s.k = {kl.batch_stride, kl.head_stride, kl.row_stride};
  s.v = {vl.batch_stride, vl.head_stride, vl.row_stride};
  s.o = {ol.batch_stride, ol.head_stride, ol.row_stride};
  return sdpa_run(ctx, B, H, Hkv, Sq, Skv, D, scale, causal, q, k, v, o, s);
}

bch_status bch_fill_uniform(bch_ctx* ctx, float* dst, size_t n, unsigned long long* state, double lo,
                            double hi) {
  if (!ctx || !state || (n && !dst)) return fail(ctx, BCH_E_INVALID, "fill_uniform: NULL argument");
  if (!(hi >= lo)) return fail(ctx, BCH_E_INVALID, "fill_uniform: hi < lo");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  st = from_hip(ctx, bch::launch_fill_uniform(ctx->stream, dst, n, *state, lo, hi), "fill_uniform launch");
  if (st == BCH_OK) *state = bch::lcg_advance(*state, 1, n);
  return st;
}

bch_status bch_fill_normal(bch_ctx* ctx, float* dst, size_t n, unsigned long long* state, double mu,
                           double sigma) {
  if (!ctx || !state || (n && !dst)) return fail(ctx, BCH_E_INVALID, "fill_normal: NULL argument");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  st = from_hip(ctx, bch::launch_fill_normal(ctx->stream, dst, n, *state, mu, sigma), "fill_normal launch");
  if (st == BCH_OK) *state = bch::lcg_advance(*state, 1442695040888963407ULL, 2 * (uint64_t)n);
  return st;
}

bch_status bch_launch_code_object(bch_ctx* ctx, const void* code_object, size_t len, const char* entry,
                                  const unsigned grid[3], const unsigned block[3], void** args, size_t nargs,
                                  size_t shared_bytes) {
  if (!ctx || !code_object || !entry || !grid || !block || (nargs && !args))
    return fail(ctx, BCH_E_INVALID, "dispatch_binary: NULL argument");
  for (int i = 0; i < 3; ++i)
    if (grid[i] == 0 || block[i] == 0)
      return fail(ctx, BCH_E_SHAPE, "dispatch_binary: zero grid/block dimension %d", i);
  if ((unsigned long long)block[0] * block[1] * block[2] > 1024)
    return fail(ctx, BCH_E_SHAPE, "dispatch_binary: block of %u x %u x %u threads exceeds 1024", block[0],
                block[1], block[2]);
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  std::string key;
  if (len == 0) {
    std::string path(static_cast<const char*>(code_object));
    if (!path.empty() && path[0] != '/') path = ctx->co_dir + "/" + path;
    key = "file:" + path;
    if (!ctx->modules.count(key)) {
      FILE* f = fopen(path.c_str(), "rb");
      if (!f) return fail(ctx, BCH_E_MODULE, "dispatch_binary: cannot open code object %s", path.c_str());
      fclose(f);
      hipModule_t mod;
      hipError_t e = hipModuleLoad(&mod, path.c_str());
      if (e != hipSuccess) return from_hip(ctx, e, "hipModuleLoad");
      ctx->modules[key] = mod;
    }
  } else {
    // Key in-memory images by address + length + a cheap content hash.
    const unsigned char* p = static_cast<const unsigned char*>(code_object);
    unsigned long long h = 1469598103934665603ULL;
    for (size_t i = 0; i < len; ++i) h = (h ^ p[i]) * 1099511628211ULL;
    char kb[64];
    snprintf(kb, sizeof(kb), "mem:%zu:%llx", len, h);
    key = kb;
    if (!ctx->modules.count(key)) {
      // A code object is an ELF image or a clang offload bundle of them;
      // reject anything else before HIP sees it.
      static const char kBundle[] = "__CLANG_OFFLOAD_BUNDLE__";
      const bool elf = len >= 4 && p[0] == 0x7f && p[1] == 'E' && p[2] == 'L' && p[3] == 'F';
      const bool bundle = len >= sizeof(kBundle) - 1 && memcmp(p, kBundle, sizeof(kBundle) - 1) == 0;
      if (!elf && !bundle)
        return fail(ctx, BCH_E_MODULE, "dispatch_binary: image is not an ELF code object");
      hipModule_t mod;
      hipError_t e = hipModuleLoadData(&mod, code_object);
      if (e != hipSuccess) return from_hip(ctx, e, "hipModuleLoadData");
      ctx->modules[key] = mod;
    }
  }
  hipFunction_t fn;
  hipError_t e = hipModuleGetFunction(&fn, ctx->modules[key], entry);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return fail(ctx, BCH_E_MODULE, "dispatch_binary: entry point '%s' not found in code object", entry);
  }
  e = hipModuleLaunchKernel(fn, grid[0], grid[1], grid[2], block[0], block[1], block[2],
                            (unsigned)shared_bytes, ctx->stream, args, nullptr);
  return from_hip(ctx, e, "hipModuleLaunchKernel");
}

bch_status bch_event_create(bch_ctx* ctx, bch_event** ev) {
  if (!ctx || !ev) return fail(ctx, BCH_E_INVALID, "bch_event_create: NULL argument");
  *ev = nullptr;
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  bch_event* x = new bch_event();
  x->device = ctx->device;
  hipError_t e = hipEventCreate(&x->ev);
  if (e != hipSuccess) {
    delete x;
    return from_hip(ctx, e, "hipEventCreate");
  }
  *ev = x;
  return BCH_OK;
}

bch_status bch_event_record(bch_ctx* ctx, bch_event* ev) {
  if (!ctx || !ev) return fail(ctx, BCH_E_INVALID, "bch_event_record: NULL argument");
  bch_status st = use(ctx);
  if (st != BCH_OK) return st;
  return from_hip(ctx, hipEventRecord(ev->ev, ctx->stream), "hipEventRecord");
}

bch_status bch_event_elapsed_ms(bch_event* start, bch_event* stop, float* ms) {
  if (!start || !stop || !ms) return fail(nullptr, BCH_E_INVALID, "bch_event_elapsed_ms: NULL argument");
  hipError_t e = hipSetDevice(stop->device);
  if (e == hipSuccess) e = hipEventSynchronize(stop->ev);
  if (e == hipSuccess) e = hipEventElapsedTime(ms, start->ev, stop->ev);
  return from_hip(nullptr, e, "hipEventElapsedTime");
}

void bch_event_destroy(bch_event* ev) {
  if (!ev) return;
  (void)hipSetDevice(ev->device);
  (void)hipEventDestroy(ev->ev);
  delete ev;
}

const char* bch_sgemm_kernel_name(int m, int n, int k) { return bch::sgemm_kernel_name(m, n, k); }

const char* bch_softmax_rows_f64_kernel_name(long long rows, long long cols, const double* in, const double* out) {
  return bch::softmax_f64_kernel_name(
      rows, cols, ((reinterpret_cast<uintptr_t>(in) | reinterpret_cast<uintptr_t>(out)) & 15) == 0);
}

const char* bch_layer_norm_kernel_name(long long rows, long long cols, const float* in, const float* out) {
  return bch::layer_norm_kernel_name(rows, cols, in, out);
}

}  // extern "C"

namespace bch {

int device_cu_count() {
  static std::atomic<int> cached[64];  // zero-initialised (static storage)
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) {
    (void)hipGetLastError();
    dev = 0;
  }
  int n = cached[dev].load(std::memory_order_relaxed);
  if (n <= 0) {
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) {
      (void)hipGetLastError();
      return kDefaultCUs;  // no device visible (validation-only calls): not cached
    }
    cached[dev].store(n, std::memory_order_relaxed);
  }
  return n;
}

hipError_t ensure_dynamic_lds(const void* func, int bytes) {
  static std::mutex mu;
  static std::set<std::tuple<const void*, int, int>> done;  // (function, device, bytes)
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> g(mu);
  const auto key = std::make_tuple(func, dev, bytes);
  if (done.count(key)) return hipSuccess;
  e = hipFuncSetAttribute(func, hipFuncAttributeMaxDynamicSharedMemorySize, bytes);
  if (e == hipSuccess) done.insert(key);
  return e;
}

}  // namespace bch
