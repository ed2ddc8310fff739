// libtl runtime: context, errors, caching allocator, copies, events and the per-launch
// event profiler. One in-order HIP stream per context; every op is enqueued on it.
#include <cstdarg>
#include <cstdlib>
#include <cstring>

#include "tl_internal.hpp"

namespace tl {

static thread_local char g_err[1024] = {0};

int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_err, sizeof(g_err), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_err[0] = 0; }

int workspace(tl_ctx* ctx, size_t bytes, void** ptr) {
  if (bytes > ctx->ws_bytes) {
    // the old buffer may still be read by queued kernels: wait for them before freeing
    TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    if (ctx->ws) (void)hipFree(ctx->ws);
    ctx->ws = nullptr;
    ctx->ws_bytes = 0;
    const size_t size = (bytes + (1u << 20) - 1) & ~(size_t)((1u << 20) - 1);
    TL_CHECK_HIP(hipMalloc(&ctx->ws, size));
    ctx->ws_bytes = size;
  }
  *ptr = ctx->ws;
  return TL_OK;
}

int enter(tl_ctx* ctx) {
  clear_error();
  if (!ctx) return fail(TL_ERR_INVALID, "null tl_ctx");
  hipError_t e = hipSetDevice(ctx->device);
  if (e != hipSuccess) return fail(TL_ERR_HIP, "hipSetDevice(%d): %s", ctx->device, hipGetErrorString(e));
  return TL_OK;
}

static hipEvent_t pool_event(tl_ctx* ctx) {
  if (!ctx->event_pool.empty()) {
    hipEvent_t e = ctx->event_pool.back();
    ctx->event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  if (hipEventCreate(&e) != hipSuccess) return nullptr;
  return e;
}

LaunchScope::LaunchScope(tl_ctx* c, int fam, double fl, double by)
    : ctx(c), family(fam), flops(fl), bytes(by) {
  if (family >= 0 && (ctx->kprof_mask & (1u << family))) {
    start = pool_event(ctx);
    if (start) (void)hipEventRecord(start, ctx->stream);
  }
}

int LaunchScope::finish(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(TL_ERR_HIP, "launch of %s failed: %s", what, hipGetErrorString(e));
  if (start) {
    hipEvent_t stop = pool_event(ctx);
    if (stop) {
      (void)hipEventRecord(stop, ctx->stream);
      ctx->kprof_pending.push_back(KprofRecord{family, start, stop, flops, bytes});
    }
  }
  return TL_OK;
}

static int kprof_drain(tl_ctx* ctx) {
  if (ctx->kprof_pending.empty()) return TL_OK;
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  for (auto& r : ctx->kprof_pending) {
    float ms = 0;
    TL_CHECK_HIP(hipEventElapsedTime(&ms, r.start, r.stop));
    KprofTotals& t = ctx->kprof_totals[r.family];
    t.launches += 1;
    t.ms += ms;
    t.flops += r.flops;
    t.bytes += r.bytes;
    ctx->event_pool.push_back(r.start);
    ctx->event_pool.push_back(r.stop);
  }
  ctx->kprof_pending.clear();
  return TL_OK;
}

static int release_cache(tl_ctx* ctx) {
  if (ctx->free_blocks.empty()) return TL_OK;
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  for (auto& kv : ctx->free_blocks) (void)hipFree(kv.second);
  ctx->free_blocks.clear();
  ctx->bytes_cached = 0;
  return TL_OK;
}

static int check_status_word(tl_ctx* ctx) {
  int32_t word = 0;
  TL_CHECK_HIP(hipMemcpy(&word, ctx->status, sizeof(word), hipMemcpyDeviceToHost));
  if (word != 0) {
    int32_t zero = 0;
    TL_CHECK_HIP(hipMemcpy(ctx->status, &zero, sizeof(zero), hipMemcpyHostToDevice));
    return fail(TL_ERR_BAD_INPUT, "a kernel saw invalid input (status 0x%x): %s", word,
                (word & 1) ? "token id out of range [0, vocab)" : "unknown");
  }
  return TL_OK;
}

}  // namespace tl

using namespace tl;

extern "C" {

int tl_version(void) { return 1; }

const char* tl_last_error(void) { return tl::g_err; }

int tl_device_count(int* count) {
  clear_error();
  TL_REQUIRE(count, "null count");
  *count = 0;
  hipError_t e = hipGetDeviceCount(count);
  if (e == hipErrorNoDevice) {
    *count = 0;
    return TL_OK;
  }
  if (e != hipSuccess) {
    *count = 0;
    return fail(TL_ERR_NO_DEVICE, "hipGetDeviceCount: %s", hipGetErrorString(e));
  }
  return TL_OK;
}

int tl_init(int device, tl_ctx** out) {
  clear_error();
  TL_REQUIRE(out, "null output pointer");
  *out = nullptr;
  int n = 0;
  hipError_t e = hipGetDeviceCount(&n);
  if (e != hipSuccess || n == 0)
    return fail(TL_ERR_NO_DEVICE, "no HIP device available (%s)",
                e == hipSuccess ? "0 devices" : hipGetErrorString(e));
  if (device < 0 || device >= n)
    return fail(TL_ERR_NO_DEVICE, "device %d out of range [0, %d)", device, n);
  TL_CHECK_HIP(hipSetDevice(device));
  hipDeviceProp_t prop;
  TL_CHECK_HIP(hipGetDeviceProperties(&prop, device));
  if (std::strncmp(prop.gcnArchName, "gfx950", 6) != 0)
    return fail(TL_ERR_UNSUPPORTED, "device %d is %s; this library is built for gfx950 only",
                device, prop.gcnArchName);
  tl_ctx* ctx = new tl_ctx();
  ctx->device = device;
  ctx->num_cus = prop.multiProcessorCount;
  if (const char* g = std::getenv("TL_GEMM_GROUP_M")) ctx->gemm_group_m = std::atoi(g);
  if (const char* g = std::getenv("TL_SKINNY_CFG")) ctx->skinny_cfg = std::atoi(g);
  if (const char* g = std::getenv("TL_SKINNY_MAX_SPLIT")) ctx->skinny_max_split = std::atoi(g);
  if (const char* g = std::getenv("TL_ATTN_DECODE_CFG")) ctx->attn_decode_cfg = std::atoi(g);
  if (const char* g = std::getenv("TL_SOFTMAX_LONG_CFG")) ctx->softmax_long_cfg = std::atoi(g);
  if (const char* g = std::getenv("TL_GEMM_TILE_FOR")) {
    long long m, n, k;
    int t, used;
    for (const char* q = g; std::sscanf(q, " %lld , %lld , %lld = %d%n", &m, &n, &k, &t, &used) == 4;) {
      ctx->tile_rules.push_back({(int64_t)m, (int64_t)n, (int64_t)k, t});
      q += used;
      while (*q == ';' || *q == ' ') ++q;
    }
  }
  e = hipStreamCreateWithFlags(&ctx->stream, hipStreamNonBlocking);
  if (e != hipSuccess) {
    delete ctx;
    return fail(TL_ERR_HIP, "hipStreamCreateWithFlags: %s", hipGetErrorString(e));
  }
  e = hipMalloc(&ctx->status, 256);
  if (e == hipSuccess) e = hipMemset(ctx->status, 0, 256);
  if (e != hipSuccess) {
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return fail(TL_ERR_HIP, "status word allocation: %s", hipGetErrorString(e));
  }
  const int src = attention_scratch_setup(ctx);
  if (src != TL_OK) {
    (void)hipFree(ctx->status);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return src;
  }
  *out = ctx;
  return TL_OK;
}

int tl_destroy(tl_ctx* ctx) {
  int rc = enter(ctx);
  if (rc) return rc;
  (void)hipStreamSynchronize(ctx->stream);
  for (auto& r : ctx->kprof_pending) {
    (void)hipEventDestroy(r.start);
    (void)hipEventDestroy(r.stop);
  }
  for (auto e : ctx->event_pool) (void)hipEventDestroy(e);
  for (auto& kv : ctx->free_blocks) (void)hipFree(kv.second);
  for (auto& kv : ctx->live) (void)hipFree(kv.first);
  (void)hipFree(ctx->status);
  if (ctx->ws) (void)hipFree(ctx->ws);
  (void)hipStreamDestroy(ctx->stream);
  delete ctx;
  return TL_OK;
}

int tl_malloc(tl_ctx* ctx, size_t bytes, void** ptr) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(ptr, "null output pointer");
  *ptr = nullptr;
  // 512-byte granularity below 1 MiB, 64 KiB above; a cached block is reused when it
  // wastes at most a quarter of itself.
  size_t size = bytes == 0 ? 512 : bytes;
  size_t gran = size < (1u << 20) ? 512 : (64u << 10);
  size = (size + gran - 1) / gran * gran;
  auto it = ctx->free_blocks.lower_bound(size);
  if (it != ctx->free_blocks.end() && it->first <= size + size / 4) {
    size_t got = it->first;
    void* p = it->second;
    ctx->free_blocks.erase(it);
    ctx->bytes_cached -= got;
    ctx->live[p] = got;
    ctx->bytes_in_use += got;
    *ptr = p;
    return TL_OK;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, size);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    rc = release_cache(ctx);
    if (rc) return rc;
    e = hipMalloc(&p, size);
    if (e != hipSuccess) {
      (void)hipGetLastError();
      return fail(TL_ERR_OOM, "hipMalloc(%zu bytes) failed: %s", size, hipGetErrorString(e));
    }
  }
  ctx->live[p] = size;
  ctx->bytes_in_use += size;
  *ptr = p;
  return TL_OK;
}

int tl_free(tl_ctx* ctx, void* ptr) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (!ptr) return TL_OK;
  auto it = ctx->live.find(ptr);
  if (it == ctx->live.end()) return fail(TL_ERR_INVALID, "tl_free: %p was not allocated by tl_malloc", ptr);
  // Stream order makes reuse safe: the next user's kernels run after this block's last
  // reader on the same stream.
  ctx->free_blocks.emplace(it->second, ptr);
  ctx->bytes_cached += it->second;
  ctx->bytes_in_use -= it->second;
  ctx->live.erase(it);
  return TL_OK;
}

int tl_empty_cache(tl_ctx* ctx) {
  int rc = enter(ctx);
  if (rc) return rc;
  return release_cache(ctx);
}

int tl_mem_stats(tl_ctx* ctx, size_t* in_use, size_t* cached) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (in_use) *in_use = ctx->bytes_in_use;
  if (cached) *cached = ctx->bytes_cached;
  return TL_OK;
}

int tl_memcpy_h2d(tl_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (bytes == 0) return TL_OK;
  TL_REQUIRE(dst && src, "null pointer");
  TL_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return TL_OK;
}

int tl_memcpy_d2h(tl_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (bytes == 0) return TL_OK;
  TL_REQUIRE(dst && src, "null pointer");
  TL_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, ctx->stream));
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return check_status_word(ctx);
}

int tl_memcpy_d2d(tl_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (bytes == 0) return TL_OK;
  TL_REQUIRE(dst && src, "null pointer");
  TL_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToDevice, ctx->stream));
  return TL_OK;
}

int tl_memcpy2d_h2d(tl_ctx* ctx, void* dst, size_t dpitch, const void* src, size_t spitch,
                    size_t width, size_t rows) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (width == 0 || rows == 0) return TL_OK;
  TL_REQUIRE(dst && src, "null pointer");
  TL_REQUIRE(width <= dpitch && width <= spitch, "width exceeds pitch");
  TL_CHECK_HIP(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, rows, hipMemcpyHostToDevice, ctx->stream));
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return TL_OK;
}

int tl_memcpy2d_d2h(tl_ctx* ctx, void* dst, size_t dpitch, const void* src, size_t spitch,
                    size_t width, size_t rows) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (width == 0 || rows == 0) return TL_OK;
  TL_REQUIRE(dst && src, "null pointer");
  TL_REQUIRE(width <= dpitch && width <= spitch, "width exceeds pitch");
  TL_CHECK_HIP(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, rows, hipMemcpyDeviceToHost, ctx->stream));
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return check_status_word(ctx);
}

int tl_sync(tl_ctx* ctx) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return check_status_word(ctx);
}

int tl_event_create(tl_ctx* ctx, void** ev) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(ev, "null output pointer");
  hipEvent_t e;
  TL_CHECK_HIP(hipEventCreate(&e));
  *ev = (void*)e;
  return TL_OK;
}

int tl_event_record(tl_ctx* ctx, void* ev) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(ev, "null event");
  TL_CHECK_HIP(hipEventRecord((hipEvent_t)ev, ctx->stream));
  return TL_OK;
}

int tl_event_elapsed_ms(void* start, void* stop, float* ms) {
  clear_error();
  TL_REQUIRE(start && stop && ms, "null argument");
  TL_CHECK_HIP(hipEventSynchronize((hipEvent_t)stop));
  TL_CHECK_HIP(hipEventElapsedTime(ms, (hipEvent_t)start, (hipEvent_t)stop));
  return TL_OK;
}

int tl_event_destroy(void* ev) {
  clear_error();
  if (!ev) return TL_OK;
  TL_CHECK_HIP(hipEventDestroy((hipEvent_t)ev));
  return TL_OK;
}

int tl_kprof_enable(tl_ctx* ctx, uint32_t mask) {
  int rc = enter(ctx);
  if (rc) return rc;
  ctx->kprof_mask = mask;
  return TL_OK;
}

int tl_kprof_reset(tl_ctx* ctx) {
  int rc = enter(ctx);
  if (rc) return rc;
  rc = kprof_drain(ctx);
  if (rc) return rc;
  for (auto& t : ctx->kprof_totals) t = KprofTotals();
  return TL_OK;
}

int tl_kprof_query(tl_ctx* ctx, int family, int64_t* launches, double* ms, double* flops,
                   double* bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(family >= 0 && family < TL_KF_COUNT, "family %d out of range", family);
  rc = kprof_drain(ctx);
  if (rc) return rc;
  const KprofTotals& t = ctx->kprof_totals[family];
  if (launches) *launches = t.launches;
  if (ms) *ms = t.ms;
  if (flops) *flops = t.flops;
  if (bytes) *bytes = t.bytes;
  return TL_OK;
}

}  // extern "C"
