// Row and elementwise kernels of the forward path: embedding gather, LayerNorm, RMSNorm,
// (causal) softmax, RoPE, GeLU/SiLU, argmax, plus fill/cast/transpose/add helpers.
//
// All of them are HBM-bound. The fast variants give one wavefront (64 lanes) to a row,
// keep the row in registers as 16-byte chunks (4 fp32 or 8 bf16 per chunk) so HBM is read
// once and written once, and reduce with cross-lane shuffles. Rows longer than a wavefront
// can hold go to a workgroup-per-row variant, and shapes whose pitch or alignment rules
// out 16-byte access use a plain scalar variant.
#include <cmath>
#include <cstring>
#include <type_traits>

#include <algorithm>

#include "tl_internal.hpp"

namespace tl {

static inline bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

static inline uint16_t host_f2bf(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

static inline unsigned grid_for(tl_ctx* ctx, int64_t work_items, int block) {
  int64_t blocks = (work_items + block - 1) / block;
  int64_t cap = (int64_t)(ctx->num_cus > 0 ? ctx->num_cus : 256) * 16;
  if (blocks > cap) blocks = cap;
  if (blocks < 1) blocks = 1;
  return (unsigned)blocks;
}

// ------------------------------------------------------------------------------------
// fill / cast / add / transpose
// ------------------------------------------------------------------------------------
template <typename T>
__global__ void fill_kernel(T* y, int64_t n, T v) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    y[i] = v;
}

template <typename TX, typename TY>
__global__ void cast_kernel(const TX* x, TY* y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    Elem<TY>::store(y + i, Elem<TX>::load(x + i));
}

// 8 elements per thread as 16-byte pieces (x and y 16-byte aligned): one 16-byte piece of
// bf16 or two of fp32 each way, raw bits when the types match; the last partial group
// element by element. One pass, no grid-stride loop: a copy of this form streams at about
// 6 TB/s on an MI355X, where the element-wise loop above reaches ~4.5.
template <typename TX, typename TY>
__global__ __launch_bounds__(256) void cast_vec_kernel(const TX* __restrict__ x, TY* __restrict__ y,
                                                       int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * 256 + threadIdx.x) * 8;
  if (i + 8 <= n) {
    if constexpr (std::is_same<TX, TY>::value) {
#pragma unroll
      for (int c = 0; c < 8 / Elem<TX>::kVec; ++c)
        reinterpret_cast<uint4*>(y + i)[c] = reinterpret_cast<const uint4*>(x + i)[c];
    } else {
      float v[8];
#pragma unroll
      for (int c = 0; c < 8 / Elem<TX>::kVec; ++c) load_chunk(x + i + c * Elem<TX>::kVec, v + c * Elem<TX>::kVec);
#pragma unroll
      for (int c = 0; c < 8 / Elem<TY>::kVec; ++c) store_chunk(y + i + c * Elem<TY>::kVec, v + c * Elem<TY>::kVec);
    }
  } else {
    for (int64_t j = i; j < n; ++j) Elem<TY>::store(y + j, Elem<TX>::load(x + j));
  }
}

template <typename T>
__global__ void add_kernel(const T* a, const T* b, T* y, int64_t n) {
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n;
       i += (int64_t)gridDim.x * blockDim.x)
    Elem<T>::store(y + i, Elem<T>::load(a + i) + Elem<T>::load(b + i));
}

// 64x64 tiles through LDS; element type is moved as raw bits.
template <typename U>
__global__ __launch_bounds__(256) void transpose_kernel(const U* x, U* y, int64_t rows,
                                                        int64_t cols, int64_t ldx, int64_t ldy) {
  __shared__ U tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    int r = ty + 4 * i;
    if (r0 + r < rows && c0 + tx < cols) tile[r][tx] = x[(r0 + r) * ldx + c0 + tx];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    int c = ty + 4 * i;
    if (c0 + c < cols && r0 + tx < rows) y[(c0 + c) * ldy + r0 + tx] = tile[tx][c];
  }
}

// The same transpose with source row r multiplied by (offset + gain[r]) on the way (an
// RMSNorm's gain folded into the K index of a packed [N, K] weight).
template <typename T>
__global__ __launch_bounds__(256) void transpose_gain_kernel(const T* x, T* y, int64_t rows,
                                                             int64_t cols, int64_t ldx,
                                                             int64_t ldy, const T* gain,
                                                             float offset) {
  __shared__ float tile[64][65];
  const int64_t r0 = (int64_t)blockIdx.y * 64, c0 = (int64_t)blockIdx.x * 64;
  const int tx = threadIdx.x & 63, ty = threadIdx.x >> 6;
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    int r = ty + 4 * i;
    if (r0 + r < rows && c0 + tx < cols)
      tile[r][tx] = Elem<T>::load(x + (r0 + r) * ldx + c0 + tx) *
                    (offset + Elem<T>::load(gain + r0 + r));
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    int c = ty + 4 * i;
    if (c0 + c < cols && r0 + tx < rows) Elem<T>::store(y + (c0 + c) * ldy + r0 + tx, tile[tx][c]);
  }
}

// ------------------------------------------------------------------------------------
// ViT patch extraction (reference transformer_adapters.py:39-47): image [B, C, H, W] ->
// tokens [B, (H/p0)(W/p1), p0 p1 C] with token index i (W/p1) + j and feature order
// (row in patch a, column in patch c2, channel ch). One thread per output element, so the
// writes are coalesced; the reads gather from the small image.
// ------------------------------------------------------------------------------------
template <typename TX, typename TY>
__global__ __launch_bounds__(256) void patchify_kernel(const TX* __restrict__ x, TY* __restrict__ y,
                                                       int64_t n, int C, int H, int W, int p0,
                                                       int p1) {
  const int pw = W / p1, L = (H / p0) * pw, tok = p0 * p1 * C;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int t = (int)(idx % tok);
    const int64_t rest = idx / tok;
    const int l = (int)(rest % L);
    const int64_t b = rest / L;
    const int ch = t % C, t2 = t / C;
    const int c2 = t2 % p1, a = t2 / p1;
    const int i = l / pw, j = l - i * pw;
    const float v = Elem<TX>::load(x + ((b * C + ch) * H + i * p0 + a) * W + j * p1 + c2);
    Elem<TY>::store(y + idx, v);
  }
}

// ------------------------------------------------------------------------------------
// embedding gather + positional add (reference transformer_adapters.py:150-151)
// ------------------------------------------------------------------------------------
template <typename T, typename I, bool VEC>
__global__ __launch_bounds__(256) void embed_kernel(const I* ids, const T* table, const T* pos,
                                                    T* out, int64_t n_tok, int64_t seq_len,
                                                    int64_t pos0, int64_t vocab, int64_t dim,
                                                    int64_t ld_out, float scale, int32_t* status) {
  constexpr int VW = Elem<T>::kVec;
  const int lane = threadIdx.x & 63;
  const int64_t tok = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= n_tok) return;
  const int64_t id = (int64_t)ids[tok];
  T* o = out + tok * ld_out;
  if (id < 0 || id >= vocab) {
    if (lane == 0) atomicOr(status, 1);
    for (int64_t c = lane; c < dim; c += 64) Elem<T>::store(o + c, 0.0f);
    return;
  }
  const T* tr = table + id * dim;
  const T* pr = pos ? pos + (pos0 + tok % seq_len) * dim : nullptr;
  if (VEC) {
    for (int64_t c = (int64_t)lane * VW; c < dim; c += 64 * VW) {
      float a[VW], b[VW];
      load_chunk(tr + c, a);
      if (scale != 1.0f) {
#pragma unroll
        for (int e = 0; e < VW; ++e) a[e] = a[e] * scale;
      }
      if (pr) {
        load_chunk(pr + c, b);
#pragma unroll
        for (int e = 0; e < VW; ++e) a[e] = a[e] + b[e];
      }
      store_chunk(o + c, a);
    }
  } else {
    for (int64_t c = lane; c < dim; c += 64) {
      float a = Elem<T>::load(tr + c);
      if (scale != 1.0f) a = a * scale;
      if (pr) a = a + Elem<T>::load(pr + c);
      Elem<T>::store(o + c, a);
    }
  }
}

// ------------------------------------------------------------------------------------
// LayerNorm / RMSNorm (reference layers.py:415-428)
// ------------------------------------------------------------------------------------
// 16-byte loads and stores, non-temporal (streamed past the caches) when NT.
template <bool NT>
__device__ __forceinline__ uint4 load16(const void* p) {
  if constexpr (NT) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(p));
    return make_uint4(t.x, t.y, t.z, t.w);
  } else {
    return *reinterpret_cast<const uint4*>(p);
  }
}
template <bool NT>
__device__ __forceinline__ void store16(void* p, const uint4& w) {
  if constexpr (NT) {
    typedef uint32_t v4u __attribute__((ext_vector_type(4)));
    const v4u t = {w.x, w.y, w.z, w.w};
    __builtin_nontemporal_store(t, reinterpret_cast<v4u*>(p));
  } else {
    *reinterpret_cast<uint4*>(p) = w;
  }
}

// Sum / maximum over a group of LPR lanes (a power of two up to 64, groups aligned to
// multiples of LPR): xor shuffles with offsets below LPR stay inside the group.
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}
template <int LPR>
__device__ __forceinline__ float group_max(float v) {
#pragma unroll
  for (int o = LPR / 2; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Norm launches with fewer workgroups than this ignore the prefetch regions (one per CU).
constexpr int kPrefetchMinGrid = 256;

// Thread `tid` of `nthreads` loads one 4-byte word of every nthreads-th 128-byte line of the
// prefetch regions, so their lines are fetched into the caches while the kernel runs; the
// words are xor-ed together and kept only so the loads are not removed.
__device__ __forceinline__ uint32_t prefetch_lines(const PrefetchList& pf, int64_t tid,
                                                   int64_t nthreads) {
  uint32_t acc = 0;
#pragma unroll
  for (int r = 0; r < 4; ++r)
    for (int64_t l = tid; l < pf.lines[r]; l += nthreads)
      acc ^= *reinterpret_cast<const uint32_t*>(pf.ptr[r] + l * 128);
  return acc;
}

// One wavefront per row, the row held in registers as raw 16-byte chunks (CH per lane),
// unpacked to float for each pass. Lanes whose chunk lies past the row end load the row's
// first chunk (a line the wave fetches anyway) and mask it out, so every load is issued
// unconditionally. LayerNorm is two-pass (mean, then squared deviations), as the reference
// computes np.var. When a lane's chunks of gamma (and beta) fit in 16 more registers
// (CH * sizeof(T) <= 16) they are loaded with the row, so their latency overlaps the row's
// instead of following the reductions. NT: the row is read and the output written
// non-temporally (the host sets it for tensors far larger than the caches, where nothing
// would be re-read from them). FULL: the row fills all CH x 64 chunks exactly, so no lane
// needs a mask (124 selects fewer per wave at bf16 x 4096).
// PF: the launch also reads the prefetch regions (a separate instantiation, so that norms
// launched without regions keep their registers: the loads issued after the row's own hold
// those registers live, 126 -> 161 VGPRs at bf16 x 4096, a wave less per SIMD).
template <typename T, int CH, bool RMS, bool NT, bool FULL, int LPR, bool PF>
__global__ __launch_bounds__(256) void norm_wave_kernel(const T* __restrict__ x,
                                                        const T* __restrict__ g,
                                                        const T* __restrict__ b,
                                                        T* __restrict__ y, int64_t rows, int cols,
                                                        int64_t ldx, int64_t ldy, float eps,
                                                        float goff, PrefetchList pf) {
  constexpr int VW = Elem<T>::kVec;
  constexpr bool PRE = CH * sizeof(T) <= 16;
  const int lane = threadIdx.x % LPR;
  const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
  if (row >= rows) return;
  const T* xr = x + row * ldx;
  uint4 raw[CH], graw[PRE ? CH : 1], braw[PRE && !RMS ? CH : 1];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * LPR + lane) * VW;
    raw[c] = load16<NT && sizeof(T) == 4>(xr + (col < cols ? col : 0));
  }
  if constexpr (PRE) {
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int col = (c * LPR + lane) * VW;
      graw[c] = *reinterpret_cast<const uint4*>(g + (col < cols ? col : 0));
      if constexpr (!RMS) braw[c] = *reinterpret_cast<const uint4*>(b + (col < cols ? col : 0));
    }
  }
  // after the row's own loads, so the waits for them do not include these
  uint32_t pf_word = 0;
  if constexpr (PF)
    pf_word = prefetch_lines(pf, (int64_t)blockIdx.x * blockDim.x + threadIdx.x,
                             (int64_t)gridDim.x * blockDim.x);
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const bool in = FULL || (c * LPR + lane) * VW < cols;
    float v[VW];
    Elem<T>::unpack(raw[c], v);
#pragma unroll
    for (int e = 0; e < VW; ++e) s += in ? (RMS ? v[e] * v[e] : v[e]) : 0.f;
  }
  float mean = 0.f, rstd;
  if (RMS) {
    rstd = 1.0f / sqrtf(group_sum<LPR>(s) / (float)cols + eps);
  } else {
    mean = group_sum<LPR>(s) / (float)cols;
    float q = 0.f;
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const bool in = FULL || (c * LPR + lane) * VW < cols;
      float v[VW];
      Elem<T>::unpack(raw[c], v);
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        const float d = v[e] - mean;
        q += in ? d * d : 0.f;
      }
    }
    rstd = 1.0f / sqrtf(group_sum<LPR>(q) / (float)cols + eps);
  }
  T* yr = y + row * ldy;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * LPR + lane) * VW;
    if (FULL || col < cols) {
      float v[VW], gv[VW], bv[VW], o[VW];
      Elem<T>::unpack(raw[c], v);
      if constexpr (PRE) {
        Elem<T>::unpack(graw[c], gv);
        if constexpr (!RMS) Elem<T>::unpack(braw[c], bv);
      } else {
        load_chunk(g + col, gv);
        if constexpr (!RMS) load_chunk(b + col, bv);
      }
#pragma unroll
      for (int e = 0; e < VW; ++e)
        o[e] = RMS ? (v[e] * rstd) * (goff + gv[e]) : gv[e] * ((v[e] - mean) * rstd) + bv[e];
      store16<NT>(yr + col, Elem<T>::pack(o));
    }
  }
  if constexpr (PF) asm volatile("" ::"v"(pf_word));
}

// Any shape: one workgroup per row, three passes over the row in global memory.
template <typename T, bool RMS>
__global__ __launch_bounds__(256) void norm_generic_kernel(const T* x, const T* g, const T* b,
                                                           T* y, int64_t rows, int64_t cols,
                                                           int64_t ldx, int64_t ldy, float eps,
                                                           float goff) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ldx;
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  auto block_sum = [&](float v) {
    v = wave_sum(v);
    __syncthreads();
    if (lane == 0) red[w] = v;
    __syncthreads();
    return red[0] + red[1] + red[2] + red[3];
  };
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float v = Elem<T>::load(xr + c);
    s += RMS ? v * v : v;
  }
  s = block_sum(s);
  float mean = 0.f, rstd;
  if (RMS) {
    rstd = 1.0f / sqrtf(s / (float)cols + eps);
  } else {
    mean = s / (float)cols;
    float q = 0.f;
    for (int64_t c = threadIdx.x; c < cols; c += 256) {
      const float d = Elem<T>::load(xr + c) - mean;
      q += d * d;
    }
    rstd = 1.0f / sqrtf(block_sum(q) / (float)cols + eps);
  }
  T* yr = y + row * ldy;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float v = Elem<T>::load(xr + c);
    const float gv = Elem<T>::load(g + c);
    const float o = RMS ? (v * rstd) * (goff + gv) : gv * ((v - mean) * rstd) + Elem<T>::load(b + c);
    Elem<T>::store(yr + c, o);
  }
}

// ------------------------------------------------------------------------------------
// softmax (reference layers.py:295-300, activations.py:57-64)
// ------------------------------------------------------------------------------------
__device__ __forceinline__ float softmax_exp(float z, float temp) {
  if (temp != 1.0f) z = z / temp;
  return __expf(z);
}

// Row r keeps columns j < valid(r); the rest are written as exact zeros (the reference's
// additive -1e9 mask underflows exp to 0). One wavefront per row, held as raw 16-byte
// chunks. Lanes whose chunk starts at or past valid(r) load the row's first chunk instead
// (a line the wave fetches anyway) and mask it out, so every load is issued unconditionally
// and a causal row reads its lower-triangle part only. TAIL: the row length is not a
// multiple of the chunk width, so the lane holding the partial last chunk loads it element
// by element.
template <typename T>
__device__ __forceinline__ uint4 load_raw_partial(const T* p, int n) {
  union {
    uint4 u;
    T e[16 / sizeof(T)];
  } r;
  r.u = make_uint4(0, 0, 0, 0);
#pragma unroll
  for (int e = 0; e < (int)(16 / sizeof(T)); ++e)
    if (e < n) r.e[e] = p[e];
  return r.u;
}

//
// exp(z / temp) is evaluated as 2^(z k) with k = log2(e) / temp, one uniform division per
// thread: a per-element z / temp compiles to a full-precision division sequence (about ten
// VALU instructions per element), and a short bf16 row is bound by VALU issue, not HBM.
// Masked elements hold -inf, so 2^((-inf - max) k) = 0 needs no per-element select.
// NTM: bit 0 makes the row loads non-temporal, bit 1 the stores (set by the host for
// tensors far larger than the caches: both for fp32, stores only for causal bf16).
template <typename T, int CH, bool CAUSAL, bool TAIL, int NTM, int LPR>
__global__ __launch_bounds__(256) void softmax_wave_kernel(const T* __restrict__ x,
                                                           T* __restrict__ y, int64_t rows,
                                                           int cols, int64_t ldx, int64_t ldy,
                                                           float temp, int64_t period,
                                                           int64_t offset) {
  constexpr int VW = Elem<T>::kVec;
  const int lane = threadIdx.x % LPR;
  const int64_t row = (int64_t)blockIdx.x * (256 / LPR) + threadIdx.x / LPR;
  if (row >= rows) return;
  int valid = cols;
  if (CAUSAL) {
    const int64_t lim = row % period + offset + 1;
    valid = lim < cols ? (int)lim : cols;
  }
  const float k = 1.4426950408889634f / temp;
  const T* xr = x + row * ldx;
  uint4 raw[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * LPR + lane) * VW;
    if (TAIL && col < valid && col + VW > cols)
      raw[c] = load_raw_partial(xr + col, cols - col);
    else
      raw[c] = load16<(NTM & 1) != 0>(xr + (col < valid ? col : 0));
  }
  float v[CH][VW];
  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * LPR + lane) * VW;
    Elem<T>::unpack(raw[c], v[c]);
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      v[c][e] = col + e < valid ? v[c][e] : -INFINITY;
      mx = fmaxf(mx, v[c][e]);
    }
  }
  mx = group_max<LPR>(mx);
  const float mref = mx == -INFINITY ? 0.f : mx;  // a row with no visible column
  float s = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      const float ex = __builtin_amdgcn_exp2f((v[c][e] - mref) * k);
      v[c][e] = ex;
      s += ex;
    }
  }
  const float rs = 1.0f / group_sum<LPR>(s);
  T* yr = y + row * ldy;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * LPR + lane) * VW;
    float o[VW];
#pragma unroll
    for (int e = 0; e < VW; ++e) o[e] = v[c][e] * rs;
    if (col + VW <= cols) {
      store16<(NTM & 2) != 0>(yr + col, Elem<T>::pack(o));
    } else if (TAIL && col < cols) {
      for (int e = 0; e < VW && col + e < cols; ++e) Elem<T>::store(yr + col + e, o[e]);
    }
  }
}

template <int NT>
__device__ __forceinline__ float block_reduce(float v, bool is_max, float* red) {
  v = is_max ? wave_max(v) : wave_sum(v);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; ++i) r = is_max ? fmaxf(r, red[i]) : r + red[i];
  return r;
}

// The packed -inf pattern of a 16-byte chunk.
template <typename T>
__device__ __forceinline__ uint4 neg_inf_chunk() {
  return sizeof(T) == 2 ? make_uint4(0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u, 0xFF80FF80u)
                        : make_uint4(0xFF800000u, 0xFF800000u, 0xFF800000u, 0xFF800000u);
}

// Long rows (vocabulary softmax, long causal rows), one workgroup of NT threads per row, the
// row held as raw 16-byte chunks (CH per thread). Each thread takes the max m_t of its own
// elements (those past the row's causal limit count as -inf and come out as 0), then
// e = 2^(k (x - m_t)) with k = log2(e) / temperature (one FMA and one exp2 per element) and
// their sum s_t; the workgroup merges the (m_t, s_t) pairs in a single reduction into the
// row's (M, S), and each thread writes e * 2^(k (m_t - M)) / S, e recomputed from the chunks.
// The row's full chunks are loaded and stored non-temporally: each logit is read once and
// each probability written once, so keeping them out of the caches leaves more room for the
// traffic in flight.
__device__ __forceinline__ void merge_max_sum(float& m, float& s, float om, float os, float k) {
  const float M = fmaxf(m, om);
  if (M == -INFINITY) return;  // both empty
  s = s * __builtin_amdgcn_exp2f((m - M) * k) + os * __builtin_amdgcn_exp2f((om - M) * k);
  m = M;
}

template <typename T, int NT, int CH, bool CAUSAL>
__global__ __launch_bounds__(NT) void softmax_long_kernel(const T* __restrict__ x,
                                                          T* __restrict__ y, int64_t rows,
                                                          int cols, int64_t ldx, int64_t ldy,
                                                          float k, int64_t period,
                                                          int64_t offset) {
  constexpr int VW = Elem<T>::kVec;
  constexpr int NW = NT / 64;
  __shared__ float wm[NW], wsum[NW];
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const T* xr = x + row * ldx;
  int valid = cols;
  if (CAUSAL) {
    const int64_t lim = row % period + offset + 1;
    valid = lim < cols ? (int)lim : cols;
  }
  // Elements at or past `valid` hold -inf: they drop out of the max, and 2^(k (-inf - m)) = 0,
  // so the passes need no per-element masks and the masked outputs are exact zeros.
  const uint4 ninf = neg_inf_chunk<T>();
  uint4 raw[CH];
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * NT + tid) * VW;
    if (c * NT * VW >= valid) {
      raw[c] = ninf;  // whole chunk past the limit (uniform)
    } else if (col + VW <= valid) {
      typedef uint32_t v4u __attribute__((ext_vector_type(4)));
      const v4u t = __builtin_nontemporal_load(reinterpret_cast<const v4u*>(xr + col));
      raw[c] = make_uint4(t.x, t.y, t.z, t.w);
    } else if (col < valid) {
      union {
        uint4 u;
        T e[VW];
      } r;
      r.u = ninf;
#pragma unroll
      for (int e = 0; e < VW; ++e)
        if (e < valid - col) r.e[e] = xr[col + e];
      raw[c] = r.u;
    } else {
      raw[c] = ninf;
    }
  }
  // The empty asm makes the packed chunks opaque between passes, so each pass unpacks them
  // again instead of keeping every unpacked float (or every exponential) live.
  auto opaque = [&]() {
#pragma unroll
    for (int c = 0; c < CH; ++c)
      asm volatile("" : "+v"(raw[c].x), "+v"(raw[c].y), "+v"(raw[c].z), "+v"(raw[c].w));
  };
  float m_t = -INFINITY;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float v[VW];
    Elem<T>::unpack(raw[c], v);
#pragma unroll
    for (int e = 0; e < VW; ++e) m_t = fmaxf(m_t, v[e]);
  }
  opaque();
  const float mk = m_t == -INFINITY ? 0.f : m_t * k;  // a thread past the row keeps e = 0
  float s_t = 0.f;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    float v[VW];
    Elem<T>::unpack(raw[c], v);
#pragma unroll
    for (int e = 0; e < VW; ++e) s_t += __builtin_amdgcn_exp2f(__builtin_fmaf(v[e], k, -mk));
  }
  opaque();
  float m = m_t, s = s_t;
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float om = __shfl_xor(m, o, 64), os = __shfl_xor(s, o, 64);
    merge_max_sum(m, s, om, os, k);
  }
  if ((tid & 63) == 0) {
    wm[tid >> 6] = m;
    wsum[tid >> 6] = s;
  }
  __syncthreads();
  float M = wm[0];
#pragma unroll
  for (int w = 1; w < NW; ++w) M = fmaxf(M, wm[w]);
  float S = 0.f;
#pragma unroll
  for (int w = 0; w < NW; ++w)
    S += wm[w] == -INFINITY ? 0.f : wsum[w] * __builtin_amdgcn_exp2f((wm[w] - M) * k);
  const float f = m_t == -INFINITY ? 0.f : __builtin_amdgcn_exp2f((m_t - M) * k) / S;
  T* yr = y + row * ldy;
#pragma unroll
  for (int c = 0; c < CH; ++c) {
    const int col = (c * NT + tid) * VW;
    if (c * NT * VW >= cols) break;  // uniform
    float o[VW];
    float v[VW];
    Elem<T>::unpack(raw[c], v);
#pragma unroll
    for (int e = 0; e < VW; ++e) o[e] = __builtin_amdgcn_exp2f(__builtin_fmaf(v[e], k, -mk)) * f;
    if (col + VW <= cols) {
      typedef uint32_t v4u __attribute__((ext_vector_type(4)));
      const uint4 w = Elem<T>::pack(o);
      const v4u t = {w.x, w.y, w.z, w.w};
      __builtin_nontemporal_store(t, reinterpret_cast<v4u*>(yr + col));
    } else if (col < cols) {
#pragma unroll
      for (int e = 0; e < VW; ++e)
        if (e < cols - col) Elem<T>::store(yr + col + e, o[e]);
    }
  }
}

// Any shape: one workgroup per row; pass 1 keeps a running (max, sum), pass 2 writes.
template <typename T, bool CAUSAL>
__global__ __launch_bounds__(256) void softmax_generic_kernel(const T* x, T* y, int64_t rows,
                                                              int64_t cols, int64_t ldx,
                                                              int64_t ldy, float temp,
                                                              int64_t period, int64_t offset) {
  __shared__ float red[4];
  const int64_t row = blockIdx.x;
  int64_t valid = cols;
  if (CAUSAL) {
    const int64_t lim = row % period + offset + 1;
    valid = lim < cols ? lim : cols;
  }
  const T* xr = x + row * ldx;
  float mx = -INFINITY;
  for (int64_t c = threadIdx.x; c < valid; c += 256) mx = fmaxf(mx, Elem<T>::load(xr + c));
  mx = block_reduce<256>(mx, true, red);
  float s = 0.f;
  for (int64_t c = threadIdx.x; c < valid; c += 256) s += softmax_exp(Elem<T>::load(xr + c) - mx, temp);
  const float r = 1.0f / block_reduce<256>(s, false, red);
  T* yr = y + row * ldy;
  for (int64_t c = threadIdx.x; c < cols; c += 256) {
    const float o = c < valid ? softmax_exp(Elem<T>::load(xr + c) - mx, temp) * r : 0.f;
    Elem<T>::store(yr + c, o);
  }
}

// ------------------------------------------------------------------------------------
// RoPE (rotate-half)
// ------------------------------------------------------------------------------------
__global__ void rope_table_kernel(float* table, int64_t seq_len, int64_t head_dim, double base,
                                  int64_t pos0) {
  const int64_t half = head_dim / 2;
  const int64_t n = seq_len * half;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = idx / half, i = idx % half;
    const double inv_freq = pow(base, -(double)(2 * i) / (double)head_dim);
    const double ang = (double)(pos0 + t) * inv_freq;
    table[idx] = (float)cos(ang);
    table[n + idx] = (float)sin(ang);
  }
}

// One sequence set of a RoPE launch: n_seq sequences of seq_len rows, seq_stride elements
// apart (x == y allowed). With row0 set, the rows start at row *row0 of each sequence (an
// int64 in device memory: a cache slice at a position known only when the kernel runs), and
// rows at or past rows_cap are left alone.
struct RopeSet {
  const void* x;
  void* y;
  int64_t n_seq, seq_stride;
  const int64_t* row0;
  int64_t rows_cap;
};

// One thread per (row, chunk of the first half): it loads that chunk and the matching chunk
// of the second half, rotates both with the position's cos/sin (from the fp32 table, read
// through L2) and writes both. Items of set 0 come first, then those of set 1 (a second
// tensor rotated by the same positions, e.g. the queries and the new cache keys of one
// attention call, so one launch serves both; n_seq = 0 leaves it empty). Item indices are
// split with 32-bit multiply-high division when the item count is below 2^31 (SMALL), else
// with 64-bit division in a grid-stride loop.
template <typename T, bool VEC, bool SMALL>
__global__ __launch_bounds__(256) void rope_kernel(RopeSet s0, RopeSet s1,
                                                   const float* __restrict__ table,
                                                   int64_t seq_len, int64_t head_dim,
                                                   FastDiv div_row, FastDiv div_seq) {
  constexpr int VW = VEC ? Elem<T>::kVec : 1;
  const int64_t half = head_dim / 2;
  const int64_t per_row = half / VW;
  const int64_t total0 = s0.n_seq * seq_len * per_row;
  const int64_t total = total0 + s1.n_seq * seq_len * per_row;
  const int64_t tsz = seq_len * half;
  auto item = [&](const RopeSet& st, int64_t i, int64_t sq, int64_t t) {
    int64_t r = t;
    if (st.row0) {
      r += *st.row0;
      if (r < t || r >= st.rows_cap) return;
    }
    const T* xr = (const T*)st.x + sq * st.seq_stride + r * head_dim;
    T* yr = (T*)st.y + sq * st.seq_stride + r * head_dim;
    const float* cs = table + t * half + i;
    const float* sn = table + tsz + t * half + i;
    float a[VW], b[VW], c[VW], s[VW], o1[VW], o2[VW];
    if (VEC) {
      load_chunk(xr + i, a);
      load_chunk(xr + half + i, b);
#pragma unroll
      for (int e = 0; e < VW; e += 4) {
        const float4 c4 = *reinterpret_cast<const float4*>(cs + e);
        const float4 s4 = *reinterpret_cast<const float4*>(sn + e);
        c[e] = c4.x; c[e + 1] = c4.y; c[e + 2] = c4.z; c[e + 3] = c4.w;
        s[e] = s4.x; s[e + 1] = s4.y; s[e + 2] = s4.z; s[e + 3] = s4.w;
      }
    } else {
      a[0] = Elem<T>::load(xr + i);
      b[0] = Elem<T>::load(xr + half + i);
      c[0] = cs[0];
      s[0] = sn[0];
    }
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      o1[e] = a[e] * c[e] - b[e] * s[e];
      o2[e] = b[e] * c[e] + a[e] * s[e];
    }
    if (VEC) {
      store_chunk(yr + i, o1);
      store_chunk(yr + half + i, o2);
    } else {
      Elem<T>::store(yr + i, o1[0]);
      Elem<T>::store(yr + half + i, o2[0]);
    }
  };
  if (SMALL) {
    uint32_t idx = blockIdx.x * 256u + threadIdx.x;
    if (idx >= (uint32_t)total) return;
    const bool second = idx >= (uint32_t)total0;
    if (second) idx -= (uint32_t)total0;
    const uint32_t row = fast_div(idx, div_row);
    const uint32_t i = (idx - row * (uint32_t)per_row) * VW;
    const uint32_t sq = fast_div(row, div_seq);
    item(second ? s1 : s0, i, sq, row - sq * (uint32_t)seq_len);
    return;
  }
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const bool second = idx >= total0;
    const int64_t j = second ? idx - total0 : idx;
    const int64_t row = j / per_row;
    const int64_t sq = row / seq_len;
    item(second ? s1 : s0, (j % per_row) * VW, sq, row - sq * seq_len);
  }
}

// ------------------------------------------------------------------------------------
// activations (reference activations.py:24-28, 41-45)
// ------------------------------------------------------------------------------------
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void act_kernel(const T* __restrict__ x, T* __restrict__ y,
                                                  int64_t n, int act) {
  constexpr int VW = VEC ? Elem<T>::kVec : 1;
  const int64_t nv = n / VW;
  for (int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; i < nv;
       i += (int64_t)gridDim.x * blockDim.x) {
    float v[VW];
    if (VEC) {
      load_chunk(x + i * VW, v);
#pragma unroll
      for (int e = 0; e < VW; ++e) v[e] = apply_act(v[e], act);
      store_chunk(y + i * VW, v);
    } else {
      Elem<T>::store(y + i, apply_act(Elem<T>::load(x + i), act));
    }
  }
  if (VEC && blockIdx.x == 0) {
    for (int64_t i = nv * VW + threadIdx.x; i < n; i += blockDim.x)
      Elem<T>::store(y + i, apply_act(Elem<T>::load(x + i), act));
  }
}

// ------------------------------------------------------------------------------------
// argmax (reference network.py:135, 158: xp.argmax(axis=-1), first index on ties)
// ------------------------------------------------------------------------------------
// True when (va, ia) should win over (vb, ib): NaN beats everything (NumPy returns the
// first NaN), then larger value, then smaller index.
__device__ __forceinline__ bool argmax_better(float va, int64_t ia, float vb, int64_t ib) {
  const bool na = va != va, nb = vb != vb;
  if (na || nb) return na && (!nb || ia < ib);
  if (va != vb) return va > vb;
  return ia < ib;
}

// One block per (row, column slice of split_len): with one slice the block writes the row's
// index; with several it writes its slice's (value, index) to pv/pi[row * slices + slice]
// and argmax_finish_kernel reduces them.
template <typename T, bool VEC>
__global__ __launch_bounds__(256) void argmax_kernel(const T* __restrict__ x, int64_t rows,
                                                     int64_t cols, int64_t ldx,
                                                     int64_t* __restrict__ out, int64_t split_len,
                                                     float* __restrict__ pv,
                                                     int64_t* __restrict__ pi) {
  constexpr int VW = VEC ? Elem<T>::kVec : 1;
  __shared__ float rv[4];
  __shared__ int64_t ri[4];
  const int64_t row = blockIdx.x;
  const T* xr = x + row * ldx;
  float best = -INFINITY;
  int64_t bi = INT64_MAX;
  const int64_t cbeg = (int64_t)blockIdx.y * split_len;
  const int64_t cend = min(cols, cbeg + split_len);
  for (int64_t c0 = cbeg + (int64_t)threadIdx.x * VW; c0 < cend; c0 += 256 * VW) {
    float v[VW];
    if (VEC && c0 + VW <= cols) {
      load_chunk(xr + c0, v);
    } else {
#pragma unroll
      for (int e = 0; e < VW; ++e) v[e] = (c0 + e < cend) ? Elem<T>::load(xr + c0 + e) : -INFINITY;
    }
#pragma unroll
    for (int e = 0; e < VW; ++e)
      if (c0 + e < cend && argmax_better(v[e], c0 + e, best, bi)) {
        best = v[e];
        bi = c0 + e;
      }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int64_t oi = __shfl_xor(bi, o, 64);
    if (argmax_better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) {
    rv[w] = best;
    ri[w] = bi;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int i = 1; i < 4; ++i)
      if (argmax_better(rv[i], ri[i], best, bi)) {
        best = rv[i];
        bi = ri[i];
      }
    if (gridDim.y == 1) {
      out[row] = bi;
    } else {
      pv[row * gridDim.y + blockIdx.y] = best;
      pi[row * gridDim.y + blockIdx.y] = bi;
    }
  }
}

// One wave per row over its `slices` (<= 64) partial results, in slice order.
__global__ __launch_bounds__(64) void argmax_finish_kernel(const float* __restrict__ pv,
                                                           const int64_t* __restrict__ pi,
                                                           int slices, int64_t* __restrict__ out) {
  const int64_t row = blockIdx.x;
  const int lane = threadIdx.x;
  float best = -INFINITY;
  int64_t bi = INT64_MAX;
  if (lane < slices) {
    best = pv[row * slices + lane];
    bi = pi[row * slices + lane];
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ov = __shfl_xor(best, o, 64);
    const int64_t oi = __shfl_xor(bi, o, 64);
    if (argmax_better(ov, oi, best, bi)) {
      best = ov;
      bi = oi;
    }
  }
  if (lane == 0) out[row] = bi;
}

}  // namespace tl

// ------------------------------------------------------------------------------------
// host-side launchers (templated on the element type)
// ------------------------------------------------------------------------------------
namespace tl {

template <typename T>
static void launch_embed(tl_ctx* ctx, int ids_dtype, const void* ids, const void* table,
                         const void* pos, void* out, int64_t n_tok, int64_t seq_len,
                         int64_t pos0, int64_t vocab, int64_t dim, int64_t ld_out, float scale) {
  const bool vec = dim % Elem<T>::kVec == 0 && ld_out % Elem<T>::kVec == 0 &&
                   aligned16(table) && aligned16(out) && (!pos || aligned16(pos));
  const unsigned g = (unsigned)((n_tok + 3) / 4);
  auto go = [&](auto id_tag) {
    typedef decltype(id_tag) I;
    if (vec)
      embed_kernel<T, I, true><<<g, 256, 0, ctx->stream>>>((const I*)ids, (const T*)table,
          (const T*)pos, (T*)out, n_tok, seq_len, pos0, vocab, dim, ld_out, scale, ctx->status);
    else
      embed_kernel<T, I, false><<<g, 256, 0, ctx->stream>>>((const I*)ids, (const T*)table,
          (const T*)pos, (T*)out, n_tok, seq_len, pos0, vocab, dim, ld_out, scale, ctx->status);
  };
  if (ids_dtype == TL_U8) go(uint8_t());
  else if (ids_dtype == TL_I32) go(int32_t());
  else go(int64_t());
}

// Lanes per row of the one-wave norm kernel: 64 (one row per wave) unless a row's 16-byte
// chunks fill 32 (or else 16) lanes exactly but not 64: then two (four) rows per wave and no
// idle lanes. The config-3 LayerNorm, bf16 [8192, 768] (96 chunks): 6.96 -> 5.94 us on hot
// operands, 9.24 -> 8.82 us rotated. The causal softmax rows (bf16 x 1024, 128 chunks) measured no gain from
// two or four rows per wave, so the softmax keeps one row per wave.
static int norm_row_lanes(int64_t chunks) {
  if (chunks % 64 == 0) return 64;
  if (chunks % 32 == 0 && chunks / 32 <= 4) return 32;
  // the ViT-S/4 LayerNorm, bf16 [33280, 384] = 48 chunks: four rows per wave, 3 chunks a lane
  if (chunks % 16 == 0 && chunks / 16 <= 4) return 16;
  return 64;
}
// Runs wave(CH, LPR) with the smallest instantiated chunks-per-lane count CH that covers a
// row of `chunks` 16-byte chunks with LPR lanes (LPR 32 or 16 only when LANES32); false when
// none does (at most MAXCH chunks per lane at 64 lanes, 4 at 32 or 16).
template <int MAXCH, bool LANES32, typename W>
static bool dispatch_row_shape(int lpr, int64_t chunks, W&& wave) {
  using std::integral_constant;
  auto at = [&](auto lpr_tag) -> bool {
    constexpr int LPR = decltype(lpr_tag)::value;
    const int64_t per = (chunks + LPR - 1) / LPR;
    if (per <= 1) wave(integral_constant<int, 1>(), lpr_tag);
    else if (per <= 2) wave(integral_constant<int, 2>(), lpr_tag);
    else if (per <= 3) wave(integral_constant<int, 3>(), lpr_tag);
    else if (per <= 4) wave(integral_constant<int, 4>(), lpr_tag);
    else if constexpr (LPR == 64) {
      if (per <= 8) wave(integral_constant<int, 8>(), lpr_tag);
      else if (MAXCH >= 16 && per <= 16) wave(integral_constant<int, MAXCH >= 16 ? 16 : 8>(), lpr_tag);
      else return false;
    } else {
      return false;
    }
    return true;
  };
  if constexpr (LANES32) {
    if (lpr == 32 && (chunks + 31) / 32 <= 4) return at(integral_constant<int, 32>());
    if (lpr == 16 && (chunks + 15) / 16 <= 4) return at(integral_constant<int, 16>());
  }
  return at(integral_constant<int, 64>());
}

template <typename T, bool RMS>
static void launch_norm(tl_ctx* ctx, const void* x, const void* g, const void* b, void* y,
                        int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, float eps,
                        float goff) {
  constexpr int VW = Elem<T>::kVec;
  const bool vec = cols % VW == 0 && ldx % VW == 0 && ldy % VW == 0 && aligned16(x) &&
                   aligned16(y) && aligned16(g) && (RMS || aligned16(b));
  const int64_t cchunks = cols / VW;  // 16-byte chunks per row
  // Rows far larger than the caches (here >= 64 MiB in) are streamed non-temporally: bf16
  // LayerNorm over [16384, 4096] 5.26 -> 5.81 TB/s with gamma/beta loaded early, fp32
  // 5.30 -> 5.75 TB/s. For bf16 only the stores are non-temporal and the loads stay cached
  // (LayerNorm 5.72 -> 6.57, RMSNorm 5.94 -> 6.57 TB/s, three same-box pairs); fp32 keeps
  // both (cached loads measured 2% slower). Smaller tensors keep cached stores, since the
  // next kernel reads them.
  const bool nt = rows * ldx * (int64_t)sizeof(T) >= ((int64_t)64 << 20);
  const bool pf = ctx->prefetch.lines[0] || ctx->prefetch.lines[1] || ctx->prefetch.lines[2] ||
                  ctx->prefetch.lines[3];
  auto wave = [&](auto ch_tag, auto lpr_tag) {
    constexpr int CH = decltype(ch_tag)::value, LPR = decltype(lpr_tag)::value;
    auto go = [&](auto nt_tag, auto full_tag) {
      constexpr bool NTV = decltype(nt_tag)::value, FULLV = decltype(full_tag)::value;
      const unsigned grid = (unsigned)((rows + 256 / LPR - 1) / (256 / LPR));
      // weights are warmed for products over in-cache activations only, so the streamed
      // (non-temporal) instantiations carry no prefetch; nor do grids of fewer workgroups
      // than CUs (a decode step's few rows): there a handful of workgroups would walk
      // megabytes of weights line by line, which the few-row product then streams anyway
      if constexpr (!NTV) {
        if (pf && grid >= (unsigned)kPrefetchMinGrid) {
          norm_wave_kernel<T, CH, RMS, false, FULLV, LPR, true><<<grid, 256, 0, ctx->stream>>>(
              (const T*)x, (const T*)g, (const T*)b, (T*)y, rows, (int)cols, ldx, ldy, eps, goff,
              ctx->prefetch);
          return;
        }
      }
      norm_wave_kernel<T, CH, RMS, NTV, FULLV, LPR, false><<<grid, 256, 0, ctx->stream>>>(
          (const T*)x, (const T*)g, (const T*)b, (T*)y, rows, (int)cols, ldx, ldy, eps, goff,
          ctx->prefetch);
    };
    const bool full = cols == (int64_t)CH * LPR * VW;
    if (nt && full) go(std::true_type(), std::true_type());
    else if (nt) go(std::true_type(), std::false_type());
    else if (full) go(std::false_type(), std::true_type());
    else go(std::false_type(), std::false_type());
  };
  const int lpr = norm_row_lanes(cchunks);
  bool done = false;
  if (vec) done = dispatch_row_shape<16, true>(lpr, cchunks, wave);
  if (!done)
    norm_generic_kernel<T, RMS><<<(unsigned)rows, 256, 0, ctx->stream>>>(
        (const T*)x, (const T*)g, (const T*)b, (T*)y, rows, cols, ldx, ldy, eps, goff);
}

template <typename T, bool CAUSAL>
static void launch_softmax(tl_ctx* ctx, const void* x, void* y, int64_t rows, int64_t cols,
                           int64_t ldx, int64_t ldy, float temp, int64_t period, int64_t offset) {
  constexpr int VW = Elem<T>::kVec;
  // masked lanes of the wave kernels read the row's first whole chunk: needs cols >= VW
  const bool vec = ldx % VW == 0 && ldy % VW == 0 && aligned16(x) && aligned16(y) && cols >= VW;
  const int64_t chunks = (cols + VW - 1) / VW;
  // Non-temporal row access for fp32 tensors far larger than the caches (causal fp32
  // [8, 12, 1024, 1024]: 5.04 -> 5.41 TB/s in a probe; the same change slowed bf16 rows).
  // Causal bf16 rows of such tensors store non-temporally and load cached (5.33 -> 5.43
  // TB/s, three same-box pairs); fp32 rows with cached loads measured no faster.
  const bool big = rows * ldx * (int64_t)sizeof(T) >= ((int64_t)64 << 20);
  const bool nt = sizeof(T) == 4 && big;
  const bool nt_store = sizeof(T) == 2 && CAUSAL && big;
  auto wave = [&](auto ch_tag, auto lpr_tag) {
    constexpr int CH = decltype(ch_tag)::value, LPR = decltype(lpr_tag)::value;
    auto go = [&](auto tail_tag, auto nt_tag) {
      constexpr bool TAIL = decltype(tail_tag)::value;
      softmax_wave_kernel<T, CH, CAUSAL, TAIL, decltype(nt_tag)::value, LPR>
          <<<(unsigned)((rows + 256 / LPR - 1) / (256 / LPR)), 256, 0, ctx->stream>>>(
              (const T*)x, (T*)y, rows, (int)cols, ldx, ldy, temp, period, offset);
    };
    if (cols % VW != 0) go(std::true_type(), std::integral_constant<int, 0>());
    else if (nt) go(std::false_type(), std::integral_constant<int, 3>());
    else if (nt_store) go(std::false_type(), std::integral_constant<int, 2>());
    else go(std::false_type(), std::integral_constant<int, 0>());
  };
  // Long rows: 512 threads for rows up to 8192 chunks (three rows resident per CU) and 1024
  // threads otherwise. On an MI355X this beat 1024 or 512 threads with e kept in registers
  // and cached loads and stores (vocabulary rows: bf16 5.10 -> 5.16 TB/s, fp32 with e kept
  // 4.51 -> 4.92 TB/s). Chunks per thread: the smallest instantiated count that covers the
  // row.
  auto longrow = [&](auto nt_tag) -> bool {
    constexpr int NT = decltype(nt_tag)::value;
    bool done = false;
    auto try_ch = [&](auto ch_tag) {
      constexpr int CH = decltype(ch_tag)::value;
      if (done || (int64_t)NT * CH < chunks) return;
      const float k = 1.4426950408889634f / temp;
      softmax_long_kernel<T, NT, CH, CAUSAL><<<(unsigned)rows, NT, 0, ctx->stream>>>(
          (const T*)x, (T*)y, rows, (int)cols, ldx, ldy, k, period, offset);
      done = true;
    };
    try_ch(std::integral_constant<int, 2>());
    try_ch(std::integral_constant<int, 4>());
    if (NT == 1024) try_ch(std::integral_constant<int, 7>());
    try_ch(std::integral_constant<int, 8>());
    try_ch(std::integral_constant<int, 13>());
    try_ch(std::integral_constant<int, 16>());
    return done;
  };
  if (vec && chunks <= 512) {
    dispatch_row_shape<8, false>(64, chunks, wave);
  } else if (vec && chunks <= 1024 * 16) {
    if (chunks <= 512 * 16) longrow(std::integral_constant<int, 512>());
    else longrow(std::integral_constant<int, 1024>());
  } else {
    softmax_generic_kernel<T, CAUSAL><<<(unsigned)rows, 256, 0, ctx->stream>>>(
        (const T*)x, (T*)y, rows, cols, ldx, ldy, temp, period, offset);
  }
}

template <typename T>
static void launch_rope(tl_ctx* ctx, const RopeSet& s0, const RopeSet& s1, const void* table,
                        int64_t seq_len, int64_t head_dim) {
  constexpr int VW = Elem<T>::kVec;
  const int64_t half = head_dim / 2;
  auto set_vec = [&](const RopeSet& st) {
    return st.n_seq == 0 ||
           (aligned16(st.x) && aligned16(st.y) && st.seq_stride % VW == 0);
  };
  const bool vec = half % VW == 0 && aligned16(table) && (seq_len * half) % 4 == 0 &&
                   set_vec(s0) && set_vec(s1);
  const int64_t work = (s0.n_seq + s1.n_seq) * seq_len * (vec ? half / VW : half);
  const bool small = work < (int64_t)0x7fffffff;
  const FastDiv dr = make_fastdiv(small ? (uint32_t)(vec ? half / VW : half) : 1u);
  const FastDiv ds = make_fastdiv(small ? (uint32_t)seq_len : 1u);
  const unsigned g = small ? (unsigned)std::max<int64_t>(1, (work + 255) / 256) : grid_for(ctx, work, 256);
  auto go = [&](auto vec_tag, auto small_tag) {
    rope_kernel<T, decltype(vec_tag)::value, decltype(small_tag)::value>
        <<<g, 256, 0, ctx->stream>>>(s0, s1, (const float*)table, seq_len, head_dim, dr, ds);
  };
  if (vec && small) go(std::true_type(), std::true_type());
  else if (vec) go(std::true_type(), std::false_type());
  else if (small) go(std::false_type(), std::true_type());
  else go(std::false_type(), std::false_type());
}

template <typename T>
static void launch_act(tl_ctx* ctx, const void* x, void* y, int64_t n, int act) {
  const bool vec = aligned16(x) && aligned16(y);
  const unsigned g = grid_for(ctx, vec ? n / Elem<T>::kVec + 1 : n, 256);
  if (vec) act_kernel<T, true><<<g, 256, 0, ctx->stream>>>((const T*)x, (T*)y, n, act);
  else act_kernel<T, false><<<g, 256, 0, ctx->stream>>>((const T*)x, (T*)y, n, act);
}

// Rows are split into column slices when there are too few rows to fill the GPU (a decode
// step's handful of vocabulary rows): slices of >= 8192 columns, at most 64 per row.
template <typename T>
static int launch_argmax(tl_ctx* ctx, const void* x, int64_t rows, int64_t cols, int64_t ldx,
                         void* out) {
  const bool vec = ldx % Elem<T>::kVec == 0 && aligned16(x);
  const int64_t target = 4LL * (ctx->num_cus > 0 ? ctx->num_cus : 256);
  int64_t slices = 1;
  if (rows < target && cols >= 2 * 8192) {
    slices = std::min<int64_t>(std::min<int64_t>((target + rows - 1) / rows, cols / 8192), 64);
    if (rows * slices > 65535LL * 64) slices = 1;
  }
  int64_t split_len = (cols + slices - 1) / slices;
  split_len = (split_len + 7) / 8 * 8;
  slices = (cols + split_len - 1) / split_len;
  float* pv = nullptr;
  int64_t* pi = nullptr;
  if (slices > 1) {
    void* ws;
    const size_t nv = (size_t)rows * slices;
    int rc = workspace(ctx, nv * (sizeof(float) + sizeof(int64_t)) + 256, &ws);
    if (rc) return rc;
    pi = (int64_t*)ws;
    pv = (float*)((char*)ws + ((nv * sizeof(int64_t) + 255) & ~(size_t)255));
  }
  const dim3 grid((unsigned)rows, (unsigned)slices);
  if (vec)
    argmax_kernel<T, true><<<grid, 256, 0, ctx->stream>>>((const T*)x, rows, cols, ldx, (int64_t*)out, split_len, pv, pi);
  else
    argmax_kernel<T, false><<<grid, 256, 0, ctx->stream>>>((const T*)x, rows, cols, ldx, (int64_t*)out, split_len, pv, pi);
  if (slices > 1)
    argmax_finish_kernel<<<(unsigned)rows, 64, 0, ctx->stream>>>(pv, pi, (int)slices, (int64_t*)out);
  return TL_OK;
}

template <bool RMS>
static int norm_entry(tl_ctx* ctx, const void* x, const void* g, const void* b, void* y,
                      int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, float eps,
                      float goff, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(dtype_is_float(dtype), "dtype %d is not a float type", dtype);
  TL_REQUIRE(rows >= 0 && cols > 0, "bad sizes");
  if (rows == 0) return TL_OK;
  TL_REQUIRE(x && g && y && (RMS || b), "null pointer");
  TL_REQUIRE(ldx >= cols && ldy >= cols, "leading dimension smaller than cols");
  TL_REQUIRE(rows < (int64_t)0x7fffffff && cols < (int64_t)0x7fffffff, "too large");
  const double es = (double)dtype_size(dtype);
  LaunchScope ls(ctx, RMS ? TL_KF_RMSNORM : TL_KF_LAYERNORM, 0,
                 es * (2.0 * rows * cols + (RMS ? 1 : 2) * cols));
  if (dtype == TL_F32) launch_norm<float, RMS>(ctx, x, g, b, y, rows, cols, ldx, ldy, eps, goff);
  else launch_norm<bf16_t, RMS>(ctx, x, g, b, y, rows, cols, ldx, ldy, eps, goff);
  ctx->prefetch = PrefetchList{};  // the hint covers one launch
  return ls.finish(RMS ? "rmsnorm_fwd" : "layernorm_fwd");
}

// out[i] = src[idx[i]] as raw elements; an index outside [0, src_len) latches bit 2 of the
// status word (reported as bad input at the next synchronising call) and writes element 0
template <typename U>
__global__ __launch_bounds__(256) void take_kernel(const U* src, int64_t src_len,
                                                   const int64_t* idx, int64_t n, U* out,
                                                   int32_t* status) {
  for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
    int64_t j = idx[i];
    if (j < 0 || j >= src_len) {
      atomicOr(status, 2);
      j = 0;
    }
    out[i] = src[j];
  }
}

}  // namespace tl

using namespace tl;

#define TL_REQUIRE_FLOAT(dtype) TL_REQUIRE(dtype_is_float(dtype), "dtype %d is not a float type", (int)(dtype))

extern "C" {

int tl_fill(tl_ctx* ctx, void* y, int64_t n, int32_t dtype, double value) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(n >= 0, "negative size");
  const size_t es = dtype_size(dtype);
  TL_REQUIRE(es, "bad dtype %d", dtype);
  if (n == 0) return TL_OK;
  TL_REQUIRE(y, "null pointer");
  LaunchScope ls(ctx, TL_KF_MISC, 0, (double)n * es);
  const unsigned g = grid_for(ctx, n, 256);
  switch (dtype) {
    case TL_F32: fill_kernel<float><<<g, 256, 0, ctx->stream>>>((float*)y, n, (float)value); break;
    case TL_BF16: fill_kernel<uint16_t><<<g, 256, 0, ctx->stream>>>((uint16_t*)y, n, host_f2bf((float)value)); break;
    case TL_I32: fill_kernel<int32_t><<<g, 256, 0, ctx->stream>>>((int32_t*)y, n, (int32_t)value); break;
    case TL_I64: fill_kernel<int64_t><<<g, 256, 0, ctx->stream>>>((int64_t*)y, n, (int64_t)value); break;
    case TL_U8: fill_kernel<uint8_t><<<g, 256, 0, ctx->stream>>>((uint8_t*)y, n, (uint8_t)value); break;
  }
  return ls.finish("fill");
}

int tl_cast(tl_ctx* ctx, const void* x, void* y, int64_t n, int32_t dx, int32_t dy) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(n >= 0, "negative size");
  TL_REQUIRE(dtype_is_float(dx) && dtype_is_float(dy), "cast supports fp32 and bf16 only");
  if (n == 0) return TL_OK;
  TL_REQUIRE(x && y, "null pointer");
  {
    const uintptr_t xa = (uintptr_t)x, ya = (uintptr_t)y;
    const uintptr_t xe = xa + (uintptr_t)n * dtype_size(dx), ye = ya + (uintptr_t)n * dtype_size(dy);
    TL_REQUIRE((dx == dy && xa == ya) || xe <= ya || ye <= xa,
               "cast operands overlap (only an in-place copy of one type is allowed)");
  }
  LaunchScope ls(ctx, TL_KF_MISC, 0, (double)n * (dtype_size(dx) + dtype_size(dy)));
  if (aligned16(x) && aligned16(y) && (n + 2047) / 2048 <= (int64_t)0xffffffffu) {
    const unsigned gv = (unsigned)((n + 2047) / 2048);
    if (dx == TL_F32 && dy == TL_BF16)
      cast_vec_kernel<float, bf16_t><<<gv, 256, 0, ctx->stream>>>((const float*)x, (bf16_t*)y, n);
    else if (dx == TL_BF16 && dy == TL_F32)
      cast_vec_kernel<bf16_t, float><<<gv, 256, 0, ctx->stream>>>((const bf16_t*)x, (float*)y, n);
    else if (dx == TL_F32)
      cast_vec_kernel<float, float><<<gv, 256, 0, ctx->stream>>>((const float*)x, (float*)y, n);
    else
      cast_vec_kernel<bf16_t, bf16_t><<<gv, 256, 0, ctx->stream>>>((const bf16_t*)x, (bf16_t*)y, n);
    return ls.finish("cast");
  }
  const unsigned g = grid_for(ctx, n, 256);
  if (dx == TL_F32 && dy == TL_BF16)
    cast_kernel<float, bf16_t><<<g, 256, 0, ctx->stream>>>((const float*)x, (bf16_t*)y, n);
  else if (dx == TL_BF16 && dy == TL_F32)
    cast_kernel<bf16_t, float><<<g, 256, 0, ctx->stream>>>((const bf16_t*)x, (float*)y, n);
  else if (dx == TL_F32)
    cast_kernel<float, float><<<g, 256, 0, ctx->stream>>>((const float*)x, (float*)y, n);
  else
    cast_kernel<bf16_t, bf16_t><<<g, 256, 0, ctx->stream>>>((const bf16_t*)x, (bf16_t*)y, n);
  return ls.finish("cast");
}

int tl_patchify(tl_ctx* ctx, const void* x, void* y, int64_t batch, int64_t channels,
                int64_t height, int64_t width, int64_t patch_h, int64_t patch_w,
                int32_t dtype_x, int32_t dtype_y) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(dtype_is_float(dtype_x) && dtype_is_float(dtype_y), "patchify supports fp32 and bf16");
  TL_REQUIRE(batch >= 0 && channels > 0 && patch_h > 0 && patch_w > 0, "bad sizes");
  TL_REQUIRE(height >= patch_h && width >= patch_w && height % patch_h == 0 && width % patch_w == 0,
             "image %lldx%lld is not a whole number of %lldx%lld patches", (long long)height,
             (long long)width, (long long)patch_h, (long long)patch_w);
  TL_REQUIRE(channels * height * width < (1LL << 31), "image too large");
  const int64_t n = batch * channels * height * width;
  if (n == 0) return TL_OK;
  TL_REQUIRE(x && y && x != y, "null or aliased pointer");
  LaunchScope ls(ctx, TL_KF_MISC, 0, (double)n * (dtype_size(dtype_x) + dtype_size(dtype_y)));
  const unsigned g = grid_for(ctx, n, 256);
  const int C = (int)channels, H = (int)height, W = (int)width, p0 = (int)patch_h, p1 = (int)patch_w;
  if (dtype_x == TL_F32 && dtype_y == TL_F32)
    patchify_kernel<float, float><<<g, 256, 0, ctx->stream>>>((const float*)x, (float*)y, n, C, H, W, p0, p1);
  else if (dtype_x == TL_F32)
    patchify_kernel<float, bf16_t><<<g, 256, 0, ctx->stream>>>((const float*)x, (bf16_t*)y, n, C, H, W, p0, p1);
  else if (dtype_y == TL_F32)
    patchify_kernel<bf16_t, float><<<g, 256, 0, ctx->stream>>>((const bf16_t*)x, (float*)y, n, C, H, W, p0, p1);
  else
    patchify_kernel<bf16_t, bf16_t><<<g, 256, 0, ctx->stream>>>((const bf16_t*)x, (bf16_t*)y, n, C, H, W, p0, p1);
  return ls.finish("patchify");
}

int tl_add(tl_ctx* ctx, const void* a, const void* b, void* y, int64_t n, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE_FLOAT(dtype);
  TL_REQUIRE(n >= 0, "negative size");
  if (n == 0) return TL_OK;
  TL_REQUIRE(a && b && y, "null pointer");
  LaunchScope ls(ctx, TL_KF_MISC, 0, 3.0 * n * dtype_size(dtype));
  const unsigned g = grid_for(ctx, n, 256);
  if (dtype == TL_F32)
    add_kernel<float><<<g, 256, 0, ctx->stream>>>((const float*)a, (const float*)b, (float*)y, n);
  else
    add_kernel<bf16_t><<<g, 256, 0, ctx->stream>>>((const bf16_t*)a, (const bf16_t*)b, (bf16_t*)y, n);
  return ls.finish("add");
}

int tl_transpose2d(tl_ctx* ctx, const void* x, void* y, int64_t rows, int64_t cols,
                   int64_t ldx, int64_t ldy, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(rows >= 0 && cols >= 0, "negative size");
  const size_t es = dtype_size(dtype);
  TL_REQUIRE(es == 2 || es == 4, "transpose supports 2- and 4-byte types");
  if (rows == 0 || cols == 0) return TL_OK;
  TL_REQUIRE(x && y && x != y, "null or aliased pointer");
  TL_REQUIRE(ldx >= cols && ldy >= rows, "leading dimension too small");
  TL_REQUIRE((cols + 63) / 64 <= 0x7fffffff && (rows + 63) / 64 <= 65535, "matrix too large");
  LaunchScope ls(ctx, TL_KF_MISC, 0, 2.0 * rows * cols * es);
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  if (es == 2)
    transpose_kernel<uint16_t><<<grid, 256, 0, ctx->stream>>>((const uint16_t*)x, (uint16_t*)y, rows, cols, ldx, ldy);
  else
    transpose_kernel<uint32_t><<<grid, 256, 0, ctx->stream>>>((const uint32_t*)x, (uint32_t*)y, rows, cols, ldx, ldy);
  return ls.finish("transpose2d");
}

int tl_take(tl_ctx* ctx, const void* src, int64_t src_len, int32_t elem_bytes,
            const int64_t* idx, int64_t n, void* out) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(elem_bytes == 1 || elem_bytes == 2 || elem_bytes == 4 || elem_bytes == 8,
             "take moves 1-, 2-, 4- or 8-byte elements");
  TL_REQUIRE(src_len > 0 && n >= 0, "bad sizes");
  if (n == 0) return TL_OK;
  TL_REQUIRE(src && idx && out, "null pointer");
  LaunchScope ls(ctx, TL_KF_MISC, 0, (8.0 + 2.0 * elem_bytes) * n);
  const unsigned g = grid_for(ctx, n, 256);
  switch (elem_bytes) {
    case 1: take_kernel<uint8_t><<<g, 256, 0, ctx->stream>>>((const uint8_t*)src, src_len, idx, n, (uint8_t*)out, ctx->status); break;
    case 2: take_kernel<uint16_t><<<g, 256, 0, ctx->stream>>>((const uint16_t*)src, src_len, idx, n, (uint16_t*)out, ctx->status); break;
    case 4: take_kernel<uint32_t><<<g, 256, 0, ctx->stream>>>((const uint32_t*)src, src_len, idx, n, (uint32_t*)out, ctx->status); break;
    default: take_kernel<uint64_t><<<g, 256, 0, ctx->stream>>>((const uint64_t*)src, src_len, idx, n, (uint64_t*)out, ctx->status); break;
  }
  return ls.finish("take");
}

int tl_transpose2d_gain(tl_ctx* ctx, const void* x, void* y, int64_t rows, int64_t cols,
                        int64_t ldx, int64_t ldy, const void* gain, float gain_offset,
                        int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE_FLOAT(dtype);
  TL_REQUIRE(rows >= 0 && cols >= 0, "negative size");
  if (rows == 0 || cols == 0) return TL_OK;
  TL_REQUIRE(x && y && gain && x != y, "null or aliased pointer");
  TL_REQUIRE(ldx >= cols && ldy >= rows, "leading dimension too small");
  TL_REQUIRE((cols + 63) / 64 <= 0x7fffffff && (rows + 63) / 64 <= 65535, "matrix too large");
  const double es = (double)dtype_size(dtype);
  LaunchScope ls(ctx, TL_KF_MISC, 0, es * (2.0 * rows * cols + rows));
  dim3 grid((unsigned)((cols + 63) / 64), (unsigned)((rows + 63) / 64));
  if (dtype == TL_F32)
    transpose_gain_kernel<float><<<grid, 256, 0, ctx->stream>>>(
        (const float*)x, (float*)y, rows, cols, ldx, ldy, (const float*)gain, gain_offset);
  else
    transpose_gain_kernel<bf16_t><<<grid, 256, 0, ctx->stream>>>(
        (const bf16_t*)x, (bf16_t*)y, rows, cols, ldx, ldy, (const bf16_t*)gain, gain_offset);
  return ls.finish("transpose2d_gain");
}

int tl_embed_fwd(tl_ctx* ctx, const void* ids, int32_t ids_dtype, const void* table,
                 const void* pos, void* out, int64_t n_tok, int64_t seq_len, int64_t pos0,
                 int64_t vocab, int64_t dim, int64_t ld_out, float scale, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE_FLOAT(dtype);
  TL_REQUIRE(n_tok >= 0 && vocab > 0 && dim > 0, "bad sizes");
  if (n_tok == 0) return TL_OK;
  TL_REQUIRE(ids && table && out, "null pointer");
  TL_REQUIRE(seq_len > 0 && pos0 >= 0 && ld_out >= dim, "bad seq_len/pos0/ld_out");
  TL_REQUIRE(ids_dtype == TL_U8 || ids_dtype == TL_I32 || ids_dtype == TL_I64, "ids must be u8, i32 or i64");
  TL_REQUIRE(n_tok / 4 + 1 < 0x7fffffff, "too many tokens");
  const double es = (double)dtype_size(dtype);
  LaunchScope ls(ctx, TL_KF_EMBED, 0,
                 (double)n_tok * (dtype_size(ids_dtype) + (pos ? 3 : 2) * dim * es));
  if (dtype == TL_F32)
    launch_embed<float>(ctx, ids_dtype, ids, table, pos, out, n_tok, seq_len, pos0, vocab, dim, ld_out, scale);
  else
    launch_embed<bf16_t>(ctx, ids_dtype, ids, table, pos, out, n_tok, seq_len, pos0, vocab, dim, ld_out, scale);
  return ls.finish("embed_fwd");
}

int tl_layernorm_fwd(tl_ctx* ctx, const void* x, const void* gamma, const void* beta, void* y,
                     int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, float eps,
                     int32_t dtype) {
  return norm_entry<false>(ctx, x, gamma, beta, y, rows, cols, ldx, ldy, eps, 0.f, dtype);
}

int tl_rmsnorm_fwd(tl_ctx* ctx, const void* x, const void* gamma, void* y, int64_t rows,
                   int64_t cols, int64_t ldx, int64_t ldy, float eps, float gamma_offset,
                   int32_t dtype) {
  return norm_entry<true>(ctx, x, gamma, nullptr, y, rows, cols, ldx, ldy, eps, gamma_offset, dtype);
}

int tl_softmax_fwd(tl_ctx* ctx, const void* x, void* y, int64_t rows, int64_t cols,
                   int64_t ldx, int64_t ldy, float temperature, int32_t causal, int64_t period,
                   int64_t offset, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE_FLOAT(dtype);
  TL_REQUIRE(rows >= 0 && cols > 0, "bad sizes");
  if (rows == 0) return TL_OK;
  TL_REQUIRE(x && y, "null pointer");
  TL_REQUIRE(ldx >= cols && ldy >= cols, "leading dimension smaller than cols");
  TL_REQUIRE(temperature > 0.f, "temperature must be positive");
  TL_REQUIRE(!causal || (period > 0 && offset >= 0), "causal softmax needs period > 0, offset >= 0");
  TL_REQUIRE(rows < (int64_t)0x7fffffff && cols < (int64_t)0x7fffffff, "too large");
  if (!causal) {
    period = 1;
    offset = 0;
  }
  // algorithmic bytes: the kept part of each row is read, the whole row written
  double kept = (double)rows * cols;
  if (causal) {
    auto tri = [&](int64_t n) {  // sum over i in [0, n) of min(cols, i + offset + 1)
      double s = 0;
      for (int64_t i = 0; i < n; ++i) s += (double)std::min<int64_t>(cols, i + offset + 1);
      return s;
    };
    kept = (double)(rows / period) * tri(period) + tri(rows % period);
  }
  const double es = (double)dtype_size(dtype);
  LaunchScope ls(ctx, TL_KF_SOFTMAX, 0, es * (kept + (double)rows * cols));
  if (dtype == TL_F32) {
    if (causal) launch_softmax<float, true>(ctx, x, y, rows, cols, ldx, ldy, temperature, period, offset);
    else launch_softmax<float, false>(ctx, x, y, rows, cols, ldx, ldy, temperature, period, offset);
  } else {
    if (causal) launch_softmax<bf16_t, true>(ctx, x, y, rows, cols, ldx, ldy, temperature, period, offset);
    else launch_softmax<bf16_t, false>(ctx, x, y, rows, cols, ldx, ldy, temperature, period, offset);
  }
  return ls.finish("softmax_fwd");
}

// Positions read from an int64 in device memory, so a captured graph replays with the
// current position rather than the one it was captured at.
__global__ void rope_table_dev_kernel(float* table, int64_t seq_len, int64_t head_dim, double base,
                                      const int64_t* pos0) {
  const int64_t half = head_dim / 2;
  const int64_t n = seq_len * half;
  const int64_t p0 = *pos0;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < n;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t t = idx / half, i = idx % half;
    const double inv_freq = pow(base, -(double)(2 * i) / (double)head_dim);
    const double ang = (double)(p0 + t) * inv_freq;
    table[idx] = (float)cos(ang);
    table[n + idx] = (float)sin(ang);
  }
}
// x[0] += delta, by lane 0 of one wave (a vector store)
__global__ void i64_add_kernel(int64_t* x, int64_t delta) {
  if (threadIdx.x == 0) x[0] = x[0] + delta;
}
// hist[r * ld + (*pos - base)] = ids[r] for r < rows when 0 <= *pos - base < cols
__global__ void ids_append_kernel(const int64_t* ids, int64_t* hist, int64_t rows, int64_t ld,
                                  int64_t cols, const int64_t* pos, int64_t base) {
  const int64_t c = *pos - base;
  if (c < 0 || c >= cols) return;
  for (int64_t r = threadIdx.x; r < rows; r += blockDim.x) hist[r * ld + c] = ids[r];
}

int tl_rope_table(tl_ctx* ctx, void* table, int64_t seq_len, int64_t head_dim, double base,
                  int64_t pos0) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(table, "null pointer");
  TL_REQUIRE(seq_len > 0 && head_dim > 0 && head_dim % 2 == 0, "head_dim must be even and positive");
  TL_REQUIRE(base > 0 && pos0 >= 0, "bad base/pos0");
  LaunchScope ls(ctx, TL_KF_MISC, 0, 4.0 * seq_len * head_dim);
  rope_table_kernel<<<grid_for(ctx, seq_len * head_dim / 2, 256), 256, 0, ctx->stream>>>(
      (float*)table, seq_len, head_dim, base, pos0);
  return ls.finish("rope_table");
}

int tl_rope_table_dev(tl_ctx* ctx, void* table, int64_t seq_len, int64_t head_dim, double base,
                      const int64_t* pos0) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(table && pos0, "null pointer");
  TL_REQUIRE(seq_len > 0 && head_dim > 0 && head_dim % 2 == 0, "head_dim must be even and positive");
  TL_REQUIRE(base > 0 && (uintptr_t)pos0 % 8 == 0, "bad base or unaligned position");
  LaunchScope ls(ctx, TL_KF_MISC, 0, 4.0 * seq_len * head_dim);
  rope_table_dev_kernel<<<grid_for(ctx, seq_len * head_dim / 2, 256), 256, 0, ctx->stream>>>(
      (float*)table, seq_len, head_dim, base, pos0);
  return ls.finish("rope_table_dev");
}

int tl_i64_add(tl_ctx* ctx, int64_t* x, int64_t delta) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(x && (uintptr_t)x % 8 == 0, "null or unaligned pointer");
  LaunchScope ls(ctx, TL_KF_MISC, 0, 16.0);
  i64_add_kernel<<<1, 64, 0, ctx->stream>>>(x, delta);
  return ls.finish("i64_add");
}

int tl_ids_append(tl_ctx* ctx, const int64_t* ids, int64_t* hist, int64_t rows, int64_t ld_hist,
                  int64_t cols, const int64_t* pos, int64_t pos_base) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(ids && hist && pos, "null pointer");
  TL_REQUIRE(rows > 0 && cols > 0 && ld_hist >= cols, "bad history shape");
  TL_REQUIRE(((uintptr_t)ids | (uintptr_t)hist | (uintptr_t)pos) % 8 == 0, "unaligned int64 operand");
  LaunchScope ls(ctx, TL_KF_MISC, 0, 16.0 * rows);
  ids_append_kernel<<<1, 256, 0, ctx->stream>>>(ids, hist, rows, ld_hist, cols, pos, pos_base);
  return ls.finish("ids_append");
}

int tl_rope_fwd(tl_ctx* ctx, const void* x, void* y, const void* table, int64_t n_seq,
                int64_t seq_len, int64_t head_dim, int64_t seq_stride, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE_FLOAT(dtype);
  TL_REQUIRE(n_seq >= 0 && seq_len > 0 && head_dim > 0 && head_dim % 2 == 0, "bad sizes");
  TL_REQUIRE(seq_stride >= seq_len * head_dim, "seq_stride < seq_len * head_dim");
  if (n_seq == 0) return TL_OK;
  TL_REQUIRE(x && y && table, "null pointer");
  const double es = (double)dtype_size(dtype);
  LaunchScope ls(ctx, TL_KF_ROPE, 0, 2.0 * es * n_seq * seq_len * head_dim);
  const RopeSet s0{x, y, n_seq, seq_stride, nullptr, 0}, s1{nullptr, nullptr, 0, 0, nullptr, 0};
  if (dtype == TL_F32) launch_rope<float>(ctx, s0, s1, table, seq_len, head_dim);
  else launch_rope<bf16_t>(ctx, s0, s1, table, seq_len, head_dim);
  return ls.finish("rope_fwd");
}

int tl_rope2_fwd(tl_ctx* ctx, const void* x1, void* y1, int64_t n_seq1, int64_t seq_stride1,
                 const void* x2, void* y2, int64_t n_seq2, int64_t seq_stride2,
                 const void* table, int64_t seq_len, int64_t head_dim, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE_FLOAT(dtype);
  TL_REQUIRE(n_seq1 >= 0 && n_seq2 >= 0 && seq_len > 0 && head_dim > 0 && head_dim % 2 == 0,
             "bad sizes");
  TL_REQUIRE((n_seq1 == 0 || seq_stride1 >= seq_len * head_dim) &&
                 (n_seq2 == 0 || seq_stride2 >= seq_len * head_dim),
             "seq_stride < seq_len * head_dim");
  if (n_seq1 + n_seq2 == 0) return TL_OK;
  TL_REQUIRE(table && (n_seq1 == 0 || (x1 && y1)) && (n_seq2 == 0 || (x2 && y2)), "null pointer");
  const double es = (double)dtype_size(dtype);
  LaunchScope ls(ctx, TL_KF_ROPE, 0, 2.0 * es * (n_seq1 + n_seq2) * seq_len * head_dim);
  const RopeSet s0{x1, y1, n_seq1, seq_stride1, nullptr, 0},
      s1{x2, y2, n_seq2, seq_stride2, nullptr, 0};
  if (dtype == TL_F32) launch_rope<float>(ctx, s0, s1, table, seq_len, head_dim);
  else launch_rope<bf16_t>(ctx, s0, s1, table, seq_len, head_dim);
  return ls.finish("rope2_fwd");
}

int tl_rope2_dev(tl_ctx* ctx, void* x1, int64_t n_seq1, int64_t seq_stride1, void* x2,
                 int64_t n_seq2, int64_t seq_stride2, int64_t rows_cap2, const void* table,
                 int64_t seq_len, int64_t head_dim, const int64_t* pos, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE_FLOAT(dtype);
  TL_REQUIRE(n_seq1 >= 0 && n_seq2 >= 0 && seq_len > 0 && head_dim > 0 && head_dim % 2 == 0,
             "bad sizes");
  TL_REQUIRE((n_seq1 == 0 || seq_stride1 >= seq_len * head_dim) &&
                 (n_seq2 == 0 || (rows_cap2 >= seq_len && seq_stride2 >= rows_cap2 * head_dim)),
             "seq_stride1 < seq_len * head_dim or seq_stride2 < rows_cap2 * head_dim");
  if (n_seq1 + n_seq2 == 0) return TL_OK;
  TL_REQUIRE(table && pos && (n_seq1 == 0 || x1) && (n_seq2 == 0 || x2), "null pointer");
  TL_REQUIRE((uintptr_t)pos % 8 == 0, "unaligned position");
  const double es = (double)dtype_size(dtype);
  LaunchScope ls(ctx, TL_KF_ROPE, 0, 2.0 * es * (n_seq1 + n_seq2) * seq_len * head_dim);
  const RopeSet s0{x1, x1, n_seq1, seq_stride1, nullptr, 0},
      s1{x2, x2, n_seq2, seq_stride2, pos, rows_cap2};
  if (dtype == TL_F32) launch_rope<float>(ctx, s0, s1, table, seq_len, head_dim);
  else launch_rope<bf16_t>(ctx, s0, s1, table, seq_len, head_dim);
  return ls.finish("rope2_dev");
}

int tl_act_fwd(tl_ctx* ctx, const void* x, void* y, int64_t n, int32_t act, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE_FLOAT(dtype);
  TL_REQUIRE(n >= 0, "negative size");
  TL_REQUIRE(act == TL_ACT_NONE || act == TL_ACT_GELU || act == TL_ACT_SILU, "bad activation %d", act);
  if (n == 0) return TL_OK;
  TL_REQUIRE(x && y, "null pointer");
  const double es = (double)dtype_size(dtype);
  LaunchScope ls(ctx, TL_KF_ACT, 0, 2.0 * es * n);
  if (dtype == TL_F32) launch_act<float>(ctx, x, y, n, act);
  else launch_act<bf16_t>(ctx, x, y, n, act);
  return ls.finish("act_fwd");
}

int tl_argmax(tl_ctx* ctx, const void* x, int64_t rows, int64_t cols, int64_t ldx,
              int32_t dtype, void* out_ids) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE_FLOAT(dtype);
  TL_REQUIRE(rows >= 0 && cols > 0, "bad sizes");
  if (rows == 0) return TL_OK;
  TL_REQUIRE(x && out_ids, "null pointer");
  TL_REQUIRE(ldx >= cols, "leading dimension smaller than cols");
  TL_REQUIRE(rows < (int64_t)0x7fffffff, "too many rows");
  LaunchScope ls(ctx, TL_KF_ARGMAX, 0, (double)dtype_size(dtype) * rows * cols + 8.0 * rows);
  rc = dtype == TL_F32 ? launch_argmax<float>(ctx, x, rows, cols, ldx, out_ids)
                      : launch_argmax<bf16_t>(ctx, x, rows, cols, ldx, out_ids);
  if (rc) return rc;
  return ls.finish("argmax");
}

}  // extern "C"
