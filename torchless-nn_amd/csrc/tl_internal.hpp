// Shared internals of libtl: the context, error reporting, launch profiling and the
// device-side helpers (bf16 conversion, 16-byte vector I/O, wavefront reductions).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdio>
#include <map>
#include <string>
#include <unordered_map>
#include <unordered_set>
#include <vector>

#include "libtl.h"

// ---------------------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------------------
namespace tl {
// Up to four device regions a kernel streams into the caches alongside its own work (one
// 4-byte load per 128-byte line, values discarded): tl_prefetch_hint.
struct PrefetchList {
  const unsigned char* ptr[4];
  int64_t lines[4];
};

// Records the message for tl_last_error() and returns `code`.
int fail(int code, const char* fmt, ...);
void clear_error();

struct KprofRecord {
  int family;
  hipEvent_t start, stop;
  double flops, bytes;
};

struct KprofTotals {
  int64_t launches = 0;
  double ms = 0, flops = 0, bytes = 0;
};

}  // namespace tl

struct tl_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  int32_t* status = nullptr;  // device word latched by kernels that see invalid data
  // caching allocator: free blocks keyed by size, live blocks by pointer
  std::multimap<size_t, void*> free_blocks;
  std::unordered_map<void*, size_t> live;
  size_t bytes_in_use = 0, bytes_cached = 0;
  // launch profiler
  uint32_t kprof_mask = 0;
  std::vector<hipEvent_t> event_pool;
  std::vector<tl::KprofRecord> kprof_pending;
  tl::KprofTotals kprof_totals[TL_KF_COUNT];
  int num_cus = 0;
  // regions named by tl_prefetch_hint, passed to the next LayerNorm / RMSNorm launch
  tl::PrefetchList prefetch{};
  // grow-only scratch for kernels that combine partial results (split argmax, split-KV
  // attention); used in stream order, so one buffer serves every call on this context
  void* ws = nullptr;
  size_t ws_bytes = 0;
  // device address, on this context's device, of the static scratch array behind
  // tl_attention_fwd_noalloc (set by tl_init), and the event recorded on this context's
  // stream after its last call that used that array
  void* noalloc_scratch = nullptr;
  hipEvent_t noalloc_done = nullptr;
  // HIP graph capture of the context stream (tl_graph_*). Blocks handed out by tl_malloc
  // while a capture is open belong to the graph it produces for as long as the graph lives:
  // its replays write them, so they are not reused even after the caller frees them.
  bool capturing = false;
  std::vector<void*> capture_blocks;             // handed out during the open capture
  std::multimap<size_t, void*> capture_free;     // freed during it (reusable by it only)
  std::unordered_map<void*, size_t> graph_block_size;  // every block a live graph holds
  std::unordered_set<void*> graph_released;      // ... that the caller has already freed
  std::vector<tl_graph*> graphs;                 // live graphs
  std::vector<void*> ws_retired;                 // workspaces replaced while graphs held them
  // stream-ordered host -> device copies: pinned staging buffers used round-robin, each
  // reusable once the copy out of it (an event) has completed
  struct Staging {
    void* host = nullptr;
    size_t bytes = 0;
    hipEvent_t done = nullptr;
    bool pending = false;
  };
  Staging staging[4];
  int staging_next = 0;
};

// A captured graph and the device blocks it holds.
struct tl_graph {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
  std::vector<void*> blocks;
};

namespace tl {

inline bool dtype_is_float(int dt) { return dt == TL_F32 || dt == TL_BF16; }
inline size_t dtype_size(int dt) {
  switch (dt) {
    case TL_F32: return 4;
    case TL_BF16: return 2;
    case TL_I32: return 4;
    case TL_I64: return 8;
    case TL_U8: return 1;
  }
  return 0;
}

// Checks the context, binds its device and clears the thread's error message.
int enter(tl_ctx* ctx);
// Returns the context's scratch buffer, grown to at least `bytes` (256-byte aligned).
int workspace(tl_ctx* ctx, size_t bytes, void** ptr);

// Looks up, once per device and with that device current, the address of the static scratch
// array behind tl_attention_fwd_noalloc, stores it in ctx->noalloc_scratch, and creates
// ctx->noalloc_done.
int attention_scratch_setup(tl_ctx* ctx);
// Takes the context out of its device's scratch turn order and destroys ctx->noalloc_done
// (tl_destroy, after the context's stream has drained).
void attention_scratch_release(tl_ctx* ctx);

// Brackets one kernel launch with profiler events when its family is enabled (a negative
// family never is: such a launch creates no events).
struct LaunchScope {
  tl_ctx* ctx;
  int family;
  double flops, bytes;
  hipEvent_t start = nullptr;
  LaunchScope(tl_ctx* c, int fam, double fl, double by);
  // Checks the launch and closes the profiler record; returns a tl_status.
  int finish(const char* what);
};

}  // namespace tl

#define TL_CHECK_HIP(expr)                                                         \
  do {                                                                             \
    hipError_t _e = (expr);                                                        \
    if (_e != hipSuccess)                                                          \
      return tl::fail(TL_ERR_HIP, "%s failed: %s", #expr, hipGetErrorString(_e));  \
  } while (0)

#define TL_REQUIRE(cond, ...)                                  \
  do {                                                         \
    if (!(cond)) return tl::fail(TL_ERR_INVALID, __VA_ARGS__); \
  } while (0)

// ---------------------------------------------------------------------------------------
// device side
// ---------------------------------------------------------------------------------------
namespace tl {

typedef uint16_t bf16_t;  // raw bf16 storage
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf2f(bf16_t v) { return __uint_as_float((uint32_t)v << 16); }
// Round-to-nearest-even (the gfx950 hardware conversion).
__device__ __forceinline__ bf16_t f2bf(float f) {
  __bf16 b = (__bf16)f;
  return __builtin_bit_cast(bf16_t, b);
}

// Division by a run-time invariant d with a multiply-high and a shift (the round-up
// method of Granlund and Montgomery, "Division by invariant integers using
// multiplication", PLDI 1994): s = ceil(log2 d), mul = floor(2^32 (2^s - d) / d) + 1,
// n / d = (mulhi(n, mul) + n) >> s for 0 <= n < 2^31.
struct FastDiv {
  uint32_t mul, shr;
};
inline FastDiv make_fastdiv(uint32_t d) {
  if (d <= 1) return FastDiv{0u, 0u};
  uint32_t s = 0;
  while ((1ull << s) < d) ++s;
  const uint64_t mul = ((1ull << 32) * ((1ull << s) - d)) / d + 1;
  return FastDiv{(uint32_t)mul, s};
}
__device__ __forceinline__ uint32_t fast_div(uint32_t n, FastDiv f) {
  return (__umulhi(n, f.mul) + n) >> f.shr;
}

template <typename T> struct Elem;
template <> struct Elem<float> {
  static constexpr int kVec = 4;  // elements per 16-byte chunk
  __device__ __forceinline__ static float load(const float* p) { return *p; }
  __device__ __forceinline__ static void store(float* p, float v) { *p = v; }
  __device__ __forceinline__ static void unpack(const uint4& u, float* v) {
    v[0] = __uint_as_float(u.x); v[1] = __uint_as_float(u.y);
    v[2] = __uint_as_float(u.z); v[3] = __uint_as_float(u.w);
  }
  __device__ __forceinline__ static uint4 pack(const float* v) {
    return make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                      __float_as_uint(v[3]));
  }
};
template <> struct Elem<bf16_t> {
  static constexpr int kVec = 8;
  __device__ __forceinline__ static float load(const bf16_t* p) { return bf2f(*p); }
  __device__ __forceinline__ static void store(bf16_t* p, float v) { *p = f2bf(v); }
  __device__ __forceinline__ static void unpack(const uint4& u, float* v) {
    const uint32_t w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[2 * i] = __uint_as_float(w[i] << 16);
      v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
  }
  __device__ __forceinline__ static uint4 pack(const float* v) {
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
      w[i] = (uint32_t)f2bf(v[2 * i]) | ((uint32_t)f2bf(v[2 * i + 1]) << 16);
    return make_uint4(w[0], w[1], w[2], w[3]);
  }
};

template <typename T>
__device__ __forceinline__ void load_chunk(const T* p, float* v) {
  Elem<T>::unpack(*reinterpret_cast<const uint4*>(p), v);
}
template <typename T>
__device__ __forceinline__ void store_chunk(T* p, const float* v) {
  *reinterpret_cast<uint4*>(p) = Elem<T>::pack(v);
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// (1 + tanh(u)) / 2 == 1 / (1 + exp(-2u)): both activations below are evaluated in this
// logistic form with the hardware exp2 and reciprocal (one transcendental each) instead of
// a tanh routine; the two forms are equal in exact arithmetic and differ by a few fp32 ulps
// of the result. exp2 overflow to +inf gives 0 and underflow to 0 gives x, the limits.
__device__ __forceinline__ float logistic_times(float x, float two_u) {
  const float e = __builtin_amdgcn_exp2f(-two_u * 1.4426950408889634f);
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}
// tanh-approximation GeLU, reference activations.py:24-28:
//   0.5 * x * (1 + tanh(sqrt(2/pi) * (x + 0.044715 * x^3)))
// With u = k (x + 0.044715 x^3), k = sqrt(2/pi): the exponent -2 u log2(e) is evaluated as
// x (c1 + c2 x^2) with c1 = -2 k log2(e), c2 = 0.044715 c1 folded (three operations).
__device__ __forceinline__ float gelu_tanh(float x) {
  const float c1 = -2.302208198144325f;    // -2 sqrt(2/pi) log2(e)
  const float c2 = -0.1029432395800235f;   // 0.044715 * c1
  const float e = __builtin_amdgcn_exp2f(x * __builtin_fmaf(c2, x * x, c1));
  return x * __builtin_amdgcn_rcpf(1.0f + e);
}
// SiLU through tanh, reference activations.py:41-45: x * (1 + tanh(x/2)) / 2
__device__ __forceinline__ float silu_tanh(float x) { return logistic_times(x, x); }
__device__ __forceinline__ float apply_act(float v, int act) {
  if (act == TL_ACT_GELU) return gelu_tanh(v);
  if (act == TL_ACT_SILU) return silu_tanh(v);
  return v;
}

// Direct global -> LDS loads (gemm.hip, attention.hip). One global_load_lds_dwordx4 through
// inline asm: each lane of the wave writes its 16 bytes at LDS base + 16 * lane, the base
// (uniform) in M0, which is saved and restored. The compiler does not track these loads, so
// it adds no wait of its own before reading the other LDS buffers (it cannot tell them apart
// and would drain every load in flight); kernels order them with dma_stage_sync, which
// waits until at most N of the wave's vector memory operations are outstanding (vmcnt counts
// loads and stores in issue order) and its LDS operations are done, then meets the other
// waves at a barrier.
__device__ __forceinline__ uint32_t lds_offset(const void* p) {
  return (uint32_t)(uintptr_t)((__attribute__((address_space(3))) const void*)p);
}
__device__ __forceinline__ void dma_load16(const void* src, uint32_t lds) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %1\n\t"
      "global_load_lds_dwordx4 %2, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "s"(lds), "v"(src)
      : "memory");
}
template <int N>
__device__ __forceinline__ void dma_stage_sync() {
  asm volatile("s_waitcnt vmcnt(%0) lgkmcnt(0)\n\ts_barrier" ::"n"(N) : "memory");
}

}  // namespace tl
