// Counter-based normal random numbers, drawn on the device (weight initialisation of
// large models without a host round trip; the reference draws on the device too when its
// runtime is CuPy, backend.py:28-31).
//
// Generator: Philox4x32-10 (Salmon, Moraes, Dror and Shaw, "Parallel random numbers: as
// easy as 1, 2, 3", SC 2011). A 128-bit counter and a 64-bit key go through 10 rounds; each
// round multiplies counter words 0 and 2 by two odd constants (32x32 -> 64 bits), mixes the
// high halves with words 1 and 3 and the key, and the key is advanced by two Weyl constants
// between rounds. Element e of a draw uses counter (e / 4, stream) and key = seed, output
// word e % 4.
// Normals: Box-Muller (Box and Muller, 1958) on the two word pairs of each counter:
//   u1 = (w0 >> 8 + 1) 2^-24 in (0, 1], u2 = (w1 >> 8) 2^-24 in [0, 1)
//   z0 = sqrt(-2 ln u1) cos(2 pi u2), z1 = sqrt(-2 ln u1) sin(2 pi u2)
// and likewise (w2, w3) -> (z2, z3); y = mean + std * z.
#include "tl_internal.hpp"

namespace tl {

struct Philox4 {
  uint32_t v[4];
};

__device__ __forceinline__ Philox4 philox4x32_10(uint32_t c0, uint32_t c1, uint32_t c2,
                                                 uint32_t c3, uint32_t k0, uint32_t k1) {
  const uint32_t mul0 = 0xD2511F53u, mul1 = 0xCD9E8D57u;
  const uint32_t weyl0 = 0x9E3779B9u, weyl1 = 0xBB67AE85u;
#pragma unroll
  for (int r = 0; r < 10; ++r) {
    const uint32_t lo0 = mul0 * c0, hi0 = __umulhi(mul0, c0);
    const uint32_t lo1 = mul1 * c2, hi1 = __umulhi(mul1, c2);
    const uint32_t n0 = hi1 ^ c1 ^ k0, n2 = hi0 ^ c3 ^ k1;
    c0 = n0; c1 = lo1; c2 = n2; c3 = lo0;
    k0 += weyl0; k1 += weyl1;
  }
  return Philox4{{c0, c1, c2, c3}};
}

__device__ __forceinline__ void box_muller(uint32_t a, uint32_t b, float& z0, float& z1) {
  const float u1 = ((float)(a >> 8) + 1.0f) * 5.9604644775390625e-08f;  // 2^-24
  const float u2 = (float)(b >> 8) * 5.9604644775390625e-08f;
  const float r = sqrtf(-2.0f * logf(u1));
  float s, c;
  sincospif(2.0f * u2, &s, &c);
  z0 = r * c;
  z1 = r * s;
}

template <typename T>
__global__ __launch_bounds__(256) void random_normal_kernel(T* y, int64_t n, uint32_t k0,
                                                            uint32_t k1, uint32_t s0,
                                                            uint32_t s1, float mean, float sd) {
  const int64_t groups = (n + 3) / 4;
  for (int64_t g = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; g < groups;
       g += (int64_t)gridDim.x * blockDim.x) {
    const Philox4 w = philox4x32_10((uint32_t)g, (uint32_t)((uint64_t)g >> 32), s0, s1, k0, k1);
    float z[4];
    box_muller(w.v[0], w.v[1], z[0], z[1]);
    box_muller(w.v[2], w.v[3], z[2], z[3]);
    const int64_t e0 = g * 4;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if (e0 + j < n) Elem<T>::store(y + e0 + j, mean + sd * z[j]);
  }
}

// Categorical sampling (the notebook's xp.random.choice(..., p=probs), demo.ipynb:1531):
// sample j draws u = (w0 >> 8) 2^-24 in [0, 1) from Philox counter (j, 0, stream) and key
// seed, and returns the smallest index i with cdf[i] > u * total, where cdf is the running
// sum of p (searchsorted(cdf, u * total, side='right')). One workgroup: thread t sums a
// contiguous chunk of p, a scan over the chunk sums in LDS gives each chunk its
// [start, end) share of [0, total), and the thread whose share holds x = u * total walks
// its chunk to the index. The walk adds the chunk's entries to `start` one by one, which
// can round below the scanned `end`; when no running sum passes x, the draw takes the
// chunk's last nonzero entry (x lies in that entry's share up to rounding), and an x at or
// past the total takes the last nonzero entry of the row, so a zero-probability index is
// never returned (the row's last index if every entry is zero).
template <typename T>
__global__ __launch_bounds__(1024) void sample_kernel(const T* p, int64_t cols, int64_t n,
                                                      uint32_t k0, uint32_t k1, uint32_t s0,
                                                      uint32_t s1, int64_t* out) {
  __shared__ float incl[1024];
  __shared__ unsigned long long last_nz;  // 1 + the row's last nonzero index (0: none)
  const int t = threadIdx.x;
  if (t == 0) last_nz = 0;
  const int64_t chunk = (cols + 1023) / 1024;
  const int64_t lo = min(cols, (int64_t)t * chunk), hi = min(cols, lo + chunk);
  float sum = 0.f;
  int64_t nz = -1;  // this chunk's last nonzero index
  for (int64_t i = lo; i < hi; ++i) {
    const float v = Elem<T>::load(p + i);
    sum += v;
    if (v != 0.f) nz = i;
  }
  incl[t] = sum;
  __syncthreads();
  if (nz >= 0) atomicMax(&last_nz, (unsigned long long)(nz + 1));
  for (int off = 1; off < 1024; off <<= 1) {  // inclusive scan (Hillis-Steele)
    const float v = t >= off ? incl[t - off] : 0.f;
    __syncthreads();
    incl[t] += v;
    __syncthreads();
  }
  const float total = incl[1023];
  const float start = t > 0 ? incl[t - 1] : 0.f, end = incl[t];
  const int64_t row_last = last_nz > 0 ? (int64_t)last_nz - 1 : cols - 1;
  for (int64_t j = 0; j < n; ++j) {
    const Philox4 w = philox4x32_10((uint32_t)j, (uint32_t)((uint64_t)j >> 32), s0, s1, k0, k1);
    const float x = (float)(w.v[0] >> 8) * 5.9604644775390625e-08f * total;
    if (x >= start && x < end) {  // a nonempty share: the chunk holds a nonzero entry
      float c = start;
      int64_t idx = nz;
      for (int64_t i = lo; i < hi; ++i) {
        c += Elem<T>::load(p + i);
        if (c > x) {
          idx = i;
          break;
        }
      }
      out[j] = idx;
    } else if (t == 1023 && !(x < total)) {
      out[j] = row_last;
    }
  }
}

}  // namespace tl

using namespace tl;

extern "C" int tl_sample(tl_ctx* ctx, const void* probs, int64_t cols, int32_t dtype, int64_t n,
                         uint64_t seed, uint64_t stream, int64_t* out) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(dtype_is_float(dtype), "sampling takes fp32 or bf16 probabilities");
  TL_REQUIRE(cols > 0 && n >= 0, "bad sizes");
  if (n == 0) return TL_OK;
  TL_REQUIRE(probs && out, "null pointer");
  LaunchScope ls(ctx, TL_KF_MISC, 0, (double)dtype_size(dtype) * cols + 8.0 * n);
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  const uint32_t s0 = (uint32_t)stream, s1 = (uint32_t)(stream >> 32);
  if (dtype == TL_F32)
    sample_kernel<float><<<1, 1024, 0, ctx->stream>>>((const float*)probs, cols, n, k0, k1, s0, s1, out);
  else
    sample_kernel<bf16_t><<<1, 1024, 0, ctx->stream>>>((const bf16_t*)probs, cols, n, k0, k1, s0, s1, out);
  return ls.finish("sample");
}

extern "C" int tl_random_normal(tl_ctx* ctx, void* y, int64_t n, uint64_t seed, uint64_t stream,
                                float mean, float std_dev, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(dtype_is_float(dtype), "random_normal supports fp32 and bf16");
  TL_REQUIRE(n >= 0, "negative size");
  if (n == 0) return TL_OK;
  TL_REQUIRE(y, "null pointer");
  const int64_t groups = (n + 3) / 4;
  int64_t blocks = (groups + 255) / 256;
  const int64_t cap = (int64_t)(ctx->num_cus > 0 ? ctx->num_cus : 256) * 32;
  if (blocks > cap) blocks = cap;
  LaunchScope ls(ctx, TL_KF_MISC, 0, (double)n * dtype_size(dtype));
  const uint32_t k0 = (uint32_t)seed, k1 = (uint32_t)(seed >> 32);
  const uint32_t s0 = (uint32_t)stream, s1 = (uint32_t)(stream >> 32);
  if (dtype == TL_F32)
    random_normal_kernel<float><<<(unsigned)blocks, 256, 0, ctx->stream>>>((float*)y, n, k0, k1, s0, s1, mean, std_dev);
  else
    random_normal_kernel<bf16_t><<<(unsigned)blocks, 256, 0, ctx->stream>>>((bf16_t*)y, n, k0, k1, s0, s1, mean, std_dev);
  return ls.finish("random_normal");
}
