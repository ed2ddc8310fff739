// libtl runtime: context, errors, caching allocator, copies, events and the per-launch
// event profiler. One in-order HIP stream per context; every op is enqueued on it.
#include <algorithm>
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
    if (ctx->capturing)
      return fail(TL_ERR_INVALID, "the workspace would grow to %zu bytes during a graph capture: "
                  "run the captured calls once before capturing them", bytes);
    // the old buffer may still be read by queued kernels: wait for them before freeing; a
    // live graph may still replay kernels that use it, so it is kept until no graph is left
    TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
    if (ctx->ws) {
      if (ctx->graphs.empty()) (void)hipFree(ctx->ws);
      else ctx->ws_retired.push_back(ctx->ws);
    }
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
  if (family >= 0 && !ctx->capturing && (ctx->kprof_mask & (1u << family))) {
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
  if (ctx->capturing) return fail(TL_ERR_INVALID, "cannot release cached blocks during a graph capture");
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
                (word & 1) ? "token id out of range [0, vocab)"
                : (word & 2) ? "gather index out of range" : "unknown");
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
  if (ctx->capturing) {
    hipGraph_t g = nullptr;
    (void)hipStreamEndCapture(ctx->stream, &g);
    if (g) (void)hipGraphDestroy(g);
    (void)hipGetLastError();
  }
  (void)hipStreamSynchronize(ctx->stream);
  attention_scratch_release(ctx);
  for (tl_graph* g : ctx->graphs) {
    (void)hipGraphExecDestroy(g->exec);
    (void)hipGraphDestroy(g->graph);
    delete g;
  }
  for (auto& kv : ctx->graph_block_size)
    if (ctx->graph_released.count(kv.first)) (void)hipFree(kv.first);
  for (void* w : ctx->ws_retired) (void)hipFree(w);
  for (auto& st : ctx->staging) {
    if (st.host) (void)hipHostFree(st.host);
    if (st.done) (void)hipEventDestroy(st.done);
  }
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
  if (ctx->capturing) {
    // a block this capture already handed out and got back is reused first (the captured
    // kernels run in stream order, as eager ones do)
    auto ct = ctx->capture_free.lower_bound(size);
    if (ct != ctx->capture_free.end() && ct->first <= size + size / 4) {
      void* p = ct->second;
      ctx->live[p] = ct->first;
      ctx->capture_free.erase(ct);
      *ptr = p;
      return TL_OK;
    }
  }
  auto it = ctx->free_blocks.lower_bound(size);
  if (it != ctx->free_blocks.end() && it->first <= size + size / 4) {
    size_t got = it->first;
    void* p = it->second;
    ctx->free_blocks.erase(it);
    ctx->bytes_cached -= got;
    ctx->live[p] = got;
    ctx->bytes_in_use += got;
    if (ctx->capturing) ctx->capture_blocks.push_back(p);
    *ptr = p;
    return TL_OK;
  }
  void* p = nullptr;
  hipError_t e = hipMalloc(&p, size);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    if (ctx->capturing)
      return fail(TL_ERR_OOM, "hipMalloc(%zu bytes) failed during a graph capture", size);
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
  if (ctx->capturing) ctx->capture_blocks.push_back(p);
  *ptr = p;
  return TL_OK;
}

int tl_free(tl_ctx* ctx, void* ptr) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (!ptr) return TL_OK;
  auto it = ctx->live.find(ptr);
  if (it == ctx->live.end()) return fail(TL_ERR_INVALID, "tl_free: %p was not allocated by tl_malloc", ptr);
  // a pending prefetch region inside this block is dropped: the block may be released to
  // the driver before the norm launch that would read it
  for (int i = 0; i < 4; ++i) {
    const unsigned char* b = (const unsigned char*)ptr;
    if (ctx->prefetch.lines[i] > 0 && ctx->prefetch.ptr[i] >= b && ctx->prefetch.ptr[i] < b + it->second)
      ctx->prefetch.lines[i] = 0;
  }
  if (ctx->graph_block_size.count(ptr)) {
    // a live graph still writes it on every replay: held until tl_graph_destroy
    ctx->graph_released.insert(ptr);
    ctx->live.erase(it);
    return TL_OK;
  }
  if (ctx->capturing &&
      std::find(ctx->capture_blocks.begin(), ctx->capture_blocks.end(), ptr) != ctx->capture_blocks.end()) {
    // handed out by the open capture: reusable by the rest of it, then held by its graph
    ctx->capture_free.emplace(it->second, ptr);
    ctx->live.erase(it);
    return TL_OK;
  }
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

int tl_workspace_bytes(tl_ctx* ctx, size_t* bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(bytes, "null pointer");
  *bytes = ctx->ws_bytes;
  return TL_OK;
}

// A pinned staging buffer of at least `bytes` whose previous copy has completed (waiting
// only for that copy), or null when the copy is too large to stage.
static constexpr size_t kStageMax = (size_t)64 << 20;
static int stage_for(tl_ctx* ctx, size_t bytes, tl_ctx::Staging** out) {
  *out = nullptr;
  if (bytes > kStageMax) return TL_OK;
  tl_ctx::Staging& st = ctx->staging[ctx->staging_next];
  ctx->staging_next = (ctx->staging_next + 1) % 4;
  if (st.pending) {
    TL_CHECK_HIP(hipEventSynchronize(st.done));
    st.pending = false;
  }
  if (!st.done) TL_CHECK_HIP(hipEventCreateWithFlags(&st.done, hipEventDisableTiming));
  if (st.bytes < bytes) {
    if (st.host) TL_CHECK_HIP(hipHostFree(st.host));
    st.host = nullptr;
    st.bytes = 0;
    const size_t sz = std::max(bytes, (size_t)1 << 20);
    TL_CHECK_HIP(hipHostMalloc(&st.host, sz, hipHostMallocDefault));
    st.bytes = sz;
  }
  *out = &st;
  return TL_OK;
}

int tl_memcpy_h2d(tl_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (bytes == 0) return TL_OK;
  TL_REQUIRE(dst && src, "null pointer");
  TL_REQUIRE(!ctx->capturing, "host copies cannot be captured in a graph");
  tl_ctx::Staging* st;
  rc = stage_for(ctx, bytes, &st);
  if (rc) return rc;
  if (st) {
    std::memcpy(st->host, src, bytes);
    TL_CHECK_HIP(hipMemcpyAsync(dst, st->host, bytes, hipMemcpyHostToDevice, ctx->stream));
    TL_CHECK_HIP(hipEventRecord(st->done, ctx->stream));
    st->pending = true;
    return TL_OK;
  }
  TL_CHECK_HIP(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, ctx->stream));
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return TL_OK;
}

int tl_memcpy_d2h(tl_ctx* ctx, void* dst, const void* src, size_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (bytes == 0) return TL_OK;
  TL_REQUIRE(dst && src, "null pointer");
  TL_REQUIRE(!ctx->capturing, "host copies cannot be captured in a graph");
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

int tl_memcpy2d_d2d(tl_ctx* ctx, void* dst, size_t dpitch, const void* src, size_t spitch,
                    size_t width, size_t rows) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (width == 0 || rows == 0) return TL_OK;
  TL_REQUIRE(dst && src, "null pointer");
  TL_REQUIRE(width <= dpitch && width <= spitch, "width exceeds pitch");
  TL_CHECK_HIP(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, rows, hipMemcpyDeviceToDevice,
                                ctx->stream));
  return TL_OK;
}

int tl_memcpy2d_h2d(tl_ctx* ctx, void* dst, size_t dpitch, const void* src, size_t spitch,
                    size_t width, size_t rows) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (width == 0 || rows == 0) return TL_OK;
  TL_REQUIRE(dst && src, "null pointer");
  TL_REQUIRE(width <= dpitch && width <= spitch, "width exceeds pitch");
  TL_REQUIRE(!ctx->capturing, "host copies cannot be captured in a graph");
  tl_ctx::Staging* st;
  rc = stage_for(ctx, width * rows, &st);
  if (rc) return rc;
  if (st) {  // rows packed into the staging buffer, then one 2D copy out of it
    for (size_t r = 0; r < rows; ++r)
      std::memcpy((char*)st->host + r * width, (const char*)src + r * spitch, width);
    TL_CHECK_HIP(hipMemcpy2DAsync(dst, dpitch, st->host, width, width, rows, hipMemcpyHostToDevice,
                                  ctx->stream));
    TL_CHECK_HIP(hipEventRecord(st->done, ctx->stream));
    st->pending = true;
    return TL_OK;
  }
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
  TL_REQUIRE(!ctx->capturing, "host copies cannot be captured in a graph");
  TL_CHECK_HIP(hipMemcpy2DAsync(dst, dpitch, src, spitch, width, rows, hipMemcpyDeviceToHost, ctx->stream));
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return check_status_word(ctx);
}

int tl_sync(tl_ctx* ctx) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(!ctx->capturing, "tl_sync during a graph capture");
  TL_CHECK_HIP(hipStreamSynchronize(ctx->stream));
  return check_status_word(ctx);
}

int tl_prefetch_hint(tl_ctx* ctx, const void* ptr, int64_t bytes) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(bytes >= 0, "negative size");
  if (bytes < 4) return TL_OK;
  TL_REQUIRE(ptr && ((uintptr_t)ptr & 3) == 0, "prefetch region must be a non-null, 4-byte aligned "
             "device pointer");
  // only memory this context handed out, so a stray pointer is an error here and never a
  // fault in the norm kernel
  bool inside = false;
  const unsigned char* p = (const unsigned char*)ptr;
  for (const auto& blk : ctx->live) {
    const unsigned char* b = (const unsigned char*)blk.first;
    if (p >= b && p < b + blk.second) {
      inside = bytes <= (int64_t)(b + blk.second - p);
      break;
    }
  }
  TL_REQUIRE(inside, "prefetch region [%p, +%lld) is not inside one live tl_malloc block", ptr,
             (long long)bytes);
  for (int i = 0; i < 4; ++i)
    if (ctx->prefetch.lines[i] == 0) {
      ctx->prefetch.ptr[i] = (const unsigned char*)ptr;
      // words at offsets 0, 128, ..., all inside [ptr, ptr + bytes)
      ctx->prefetch.lines[i] = (bytes - 4) / 128 + 1;
      return TL_OK;
    }
  return fail(TL_ERR_INVALID, "at most 4 prefetch regions may wait for the next norm launch");
}

int tl_graph_begin(tl_ctx* ctx) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(!ctx->capturing, "a graph capture is already open on this context");
  TL_CHECK_HIP(hipStreamBeginCapture(ctx->stream, hipStreamCaptureModeRelaxed));
  ctx->capturing = true;
  ctx->capture_blocks.clear();
  ctx->capture_free.clear();
  return TL_OK;
}

// Ends the open capture; the blocks it handed out become held by `g` (or, when the capture
// failed, go back to the cache: the caller's, once freed, and those freed during it).
static void settle_capture_blocks(tl_ctx* ctx, tl_graph* g) {
  std::unordered_set<void*> freed;
  for (auto& kv : ctx->capture_free) freed.insert(kv.second);
  for (void* b : ctx->capture_blocks) {
    size_t sz = 0;
    auto lv = ctx->live.find(b);
    if (lv != ctx->live.end()) sz = lv->second;
    for (auto& kv : ctx->capture_free)
      if (kv.second == b) sz = kv.first;
    if (g) {
      g->blocks.push_back(b);
      ctx->graph_block_size[b] = sz;
      if (freed.count(b)) ctx->graph_released.insert(b);
    } else if (freed.count(b)) {
      ctx->free_blocks.emplace(sz, b);
      ctx->bytes_cached += sz;
      ctx->bytes_in_use -= sz;
    }
  }
  ctx->capture_blocks.clear();
  ctx->capture_free.clear();
}

int tl_graph_end(tl_ctx* ctx, tl_graph** out) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(out, "null output pointer");
  *out = nullptr;
  TL_REQUIRE(ctx->capturing, "no graph capture is open on this context");
  hipGraph_t graph = nullptr;
  hipError_t e = hipStreamEndCapture(ctx->stream, &graph);
  ctx->capturing = false;
  hipGraphExec_t exec = nullptr;
  if (e == hipSuccess && graph) e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
  if (e != hipSuccess || !graph) {
    if (graph) (void)hipGraphDestroy(graph);
    (void)hipGetLastError();
    settle_capture_blocks(ctx, nullptr);
    return fail(TL_ERR_HIP, "graph capture failed: %s", hipGetErrorString(e));
  }
  tl_graph* g = new tl_graph();
  g->graph = graph;
  g->exec = exec;
  settle_capture_blocks(ctx, g);
  ctx->graphs.push_back(g);
  *out = g;
  return TL_OK;
}

int tl_graph_launch(tl_ctx* ctx, tl_graph* g) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(g && std::find(ctx->graphs.begin(), ctx->graphs.end(), g) != ctx->graphs.end(),
             "not a live graph of this context");
  TL_REQUIRE(!ctx->capturing, "graph launch during a graph capture");
  TL_CHECK_HIP(hipGraphLaunch(g->exec, ctx->stream));
  return TL_OK;
}

int tl_graph_destroy(tl_ctx* ctx, tl_graph* g) {
  int rc = enter(ctx);
  if (rc) return rc;
  if (!g) return TL_OK;
  auto it = std::find(ctx->graphs.begin(), ctx->graphs.end(), g);
  TL_REQUIRE(it != ctx->graphs.end(), "not a live graph of this context");
  ctx->graphs.erase(it);
  // replays still queued finish before the executable goes
  const hipError_t se = hipStreamSynchronize(ctx->stream);
  (void)hipGraphExecDestroy(g->exec);
  (void)hipGraphDestroy(g->graph);
  // blocks the caller has freed return to the cache (stream order: later users run after
  // the graph's last queued replay); blocks the caller still holds stay its own
  for (void* b : g->blocks) {
    const size_t sz = ctx->graph_block_size[b];
    ctx->graph_block_size.erase(b);
    if (ctx->graph_released.erase(b)) {
      ctx->free_blocks.emplace(sz, b);
      ctx->bytes_cached += sz;
      ctx->bytes_in_use -= sz;
    }
  }
  delete g;
  if (ctx->graphs.empty() && !ctx->ws_retired.empty()) {
    for (void* w : ctx->ws_retired) (void)hipFree(w);
    ctx->ws_retired.clear();
  }
  if (se != hipSuccess) return fail(TL_ERR_HIP, "stream synchronize: %s", hipGetErrorString(se));
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
