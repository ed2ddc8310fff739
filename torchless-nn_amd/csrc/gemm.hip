// GEMMs of the forward path: C = epilogue(A * op(B)), batched and strided.
//
// gemm_mfma_kernel: bf16 operands, fp32 accumulation on the gfx950 matrix cores
//   (v_mfma_f32_16x16x32_bf16). A is [M, K] and B is given K-contiguous as Bt [N, K], so
//   both tiles stream from memory as 16-byte chunks of K. Four wavefronts split a BM x BN
//   output tile 2 x 2; each holds a (BM/2) x (BN/2) accumulator block, up to 128 x 128 (256
//   fp32 accumulators per lane) so that one K step of 64 is 128 MFMAs per wave, long enough
//   to cover the latency of the next step's global loads, which are issued before it.
//   Operand tiles are double-buffered in LDS (one barrier per K step); the 16-byte chunks
//   of a row are XOR-swizzled by row so fragment reads of 16 consecutive rows hit distinct
//   banks. The MFMA takes Bt as its first operand, so each lane's 4 results are 4
//   consecutive output columns of one row, stored as one 8- or 16-byte write.
//   Output tiles are visited in an XCD-aware grouped order: workgroups are dispatched
//   round-robin over the 8 XCDs, so block ids are remapped to give every XCD a contiguous
//   run of tiles, and tiles run in groups of a few tile-rows (group_m) so the A and B panels
//   a group shares stay in that XCD's L2.
// gemm_simt_kernel: any dtype, layout or alignment, fp32 FMA on the vector ALUs. It
//   serves the fp32 model and shapes the MFMA kernel's 16-byte loads cannot take.
#include <algorithm>

#include "tl_internal.hpp"

namespace tl {

// Epilogues of the LDS-staged path, one compiled variant each (bias, activation and
// residual known at compile time, so the fragment loops carry no per-element tests);
// EPI_GENERIC keeps mfma_epilogue (QKV scatter, GeGLU, fp32 output, divisor, unaligned
// residual rows or output rows).
enum EpiKind { EPI_GENERIC = 0, EPI_PLAIN, EPI_BIAS, EPI_BIAS_GELU, EPI_BIAS_SILU, EPI_BIAS_RES, EPI_RES,
               EPI_QKV, EPI_QKV_BIAS, EPI_GEGLU_GELU, EPI_GEGLU_SILU };

struct GemmParams {
  const void* A;
  const void* B;
  void* C;
  int64_t M, N, K, lda, ldb, ldc;
  int64_t batch_inner;
  int64_t sa_o, sa_i, sb_o, sb_i, sc_o, sc_i;
  const void* bias;
  const void* res;
  int64_t ldr, sr_o, sr_i;
  float divisor;
  int act;
  int b_kn;
  int vec_store;
  int vec_res;  // residual rows allow one 4-element vector load per lane fragment
  int epi;      // EpiKind: which specialised LDS-staged epilogue applies (bf16 output)
  int qkv;
  void* q;
  void* k;
  void* vt;
  int T, Hq, Hkv, Dh;
  int L, pos0;  // key/value cache capacity and write position (QKV split)
  const int64_t* pos0_dev;  // when set: the write position, read from device memory
  int geglu;    // gated epilogue: C[m, n/2] = act(acc[m, n]) * acc[m, n+1]
  int tiles_m, tiles_n, group_m;
  FastDiv div_T, div_Dh;
  // RMS row scaling (skinny kernel): the product of row m is multiplied by
  // 1 / sqrt(sum_k A[m, k]^2 / K + norm_eps) before the epilogue, which with the norm's gain
  // folded into B makes it RMSNorm(A) @ B
  int norm_rows;
  float norm_eps;
};

// Global-memory access through an address-space-1 pointer. The epilogue's pointers come
// from the parameter block, so the compiler cannot prove they are global and would emit
// flat instructions, which also count in the LDS wait counter: every wait for an LDS read
// would then wait for the stores issued before it as well.
// (HIP's uint2/uint4 are C++ structs whose assignment takes a generic `this`, so 8- and
// 16-byte accesses go through native vector types.)
template <typename T>
__device__ __forceinline__ void gstore(T* p, const T& v) {
  *(__attribute__((address_space(1))) T*)p = v;
}
template <typename T>
__device__ __forceinline__ T gload(const T* p) {
  return *(const __attribute__((address_space(1))) T*)p;
}
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void gstore16(void* p, uint4 v) {
  const u32x4_t t = {v.x, v.y, v.z, v.w};
  *(__attribute__((address_space(1))) u32x4_t*)p = t;
}
__device__ __forceinline__ void gstore8(void* p, uint2 v) {
  const u32x2_t t = {v.x, v.y};
  *(__attribute__((address_space(1))) u32x2_t*)p = t;
}
__device__ __forceinline__ uint2 gload8(const void* p) {
  const u32x2_t t = *(const __attribute__((address_space(1))) u32x2_t*)p;
  return make_uint2(t.x, t.y);
}
template <typename T>
__device__ __forceinline__ void gstore_elem(T* p, float v) {
  if (sizeof(T) == 4) gstore(reinterpret_cast<float*>(p), v);
  else gstore(reinterpret_cast<bf16_t*>(p), f2bf(v));
}
template <typename T>
__device__ __forceinline__ float gload_elem(const T* p) {
  if (sizeof(T) == 4) return gload(reinterpret_cast<const float*>(p));
  return bf2f(gload(reinterpret_cast<const bf16_t*>(p)));
}
__device__ __forceinline__ void gstore_f4(float* p, const float (&v)[4]) {
  gstore16(p, make_uint4(__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]),
                         __float_as_uint(v[3])));
}
__device__ __forceinline__ void gload_f4(const float* p, float (&v)[4]) {
  const u32x4_t t = *(const __attribute__((address_space(1))) u32x4_t*)p;
  v[0] = __uint_as_float(t.x); v[1] = __uint_as_float(t.y);
  v[2] = __uint_as_float(t.z); v[3] = __uint_as_float(t.w);
}

// Bias value of column n, 0 past N. The load itself is unconditional (column clamped to
// N - 1) and the value is selected afterwards: a load under a per-lane condition compiles to
// its own exec-masked branch that waits for it, so a fragment's loads would complete one
// after another instead of together.
__device__ __forceinline__ float bias_at(const GemmParams& e, int64_t n) {
  const float b = bf2f(gload((const bf16_t*)e.bias + (n < e.N ? n : e.N - 1)));
  return n < e.N ? b : 0.f;
}

// Applies the epilogue to 4 consecutive columns n0..n0+3 of row m and stores them.
template <typename TI, typename TO>
__device__ __forceinline__ void epilogue4(const GemmParams& p, int64_t zo, int64_t zi, int64_t m,
                                          int64_t n0, float v[4]) {
  if (m >= p.M || n0 >= p.N) return;
  const int cnt = p.N - n0 >= 4 ? 4 : (int)(p.N - n0);
  if (p.divisor != 1.0f) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = v[e] / p.divisor;
  }
  if (p.bias) {  // unconditional loads (clamped to column N - 1), selected afterwards
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float b = gload_elem((const TI*)p.bias + (e < cnt ? n0 + e : p.N - 1));
      if (e < cnt) v[e] = v[e] + b;
    }
  }
  if (p.geglu) {  // columns (gate f, up f, gate f+1, up f+1), n0 even
    TO* c = (TO*)p.C + zo * p.sc_o + zi * p.sc_i + m * p.ldc + n0 / 2;
    gstore_elem(c, apply_act(v[0], p.act) * v[1]);
    if (cnt == 4) gstore_elem(c + 1, apply_act(v[2], p.act) * v[3]);
    return;
  }
  if (p.act != TL_ACT_NONE) {
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = apply_act(v[e], p.act);
  }
  if (p.res) {
    const TO* r = (const TO*)p.res + zo * p.sr_o + zi * p.sr_i + m * p.ldr;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float x = gload_elem(r + (e < cnt ? n0 + e : p.N - 1));
      if (e < cnt) v[e] = v[e] + x;
    }
  }
  if (p.qkv) {
    // Dh % 4 == 0 (checked on the host), so the 4 columns share one head of one part.
    const int mi = (int)m, ni = (int)n0;
    const int b = mi / p.T, t = mi - b * p.T;
    const int pos0 = p.pos0_dev ? (int)*p.pos0_dev : p.pos0;
    const int qw = p.Hq * p.Dh, kw = p.Hkv * p.Dh;
    TO* dst;
    int64_t step;
    if (ni < qw) {
      const int h = ni / p.Dh, d = ni - h * p.Dh;
      dst = (TO*)p.q + ((int64_t)(b * p.Hq + h) * p.T + t) * p.Dh + d;
      step = 1;
    } else if (ni < qw + kw) {
      if (t + pos0 >= p.L) return;  // a device position past the cache: nothing written
      const int nn = ni - qw, h = nn / p.Dh, d = nn - h * p.Dh;
      dst = (TO*)p.k + ((int64_t)(b * p.Hkv + h) * p.L + t + pos0) * p.Dh + d;
      step = 1;
    } else {
      if (t + pos0 >= p.L) return;
      const int nn = ni - qw - kw, h = nn / p.Dh, d = nn - h * p.Dh;
      dst = (TO*)p.vt + ((int64_t)(b * p.Hkv + h) * p.Dh + d) * p.L + t + pos0;
      step = p.L;
    }
    if (step == 1 && sizeof(TO) == 2) {
      uint2 w;
      w.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
      w.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
      gstore8(dst, w);
    } else {
#pragma unroll
      for (int e = 0; e < 4; ++e) gstore_elem(dst + e * step, v[e]);
    }
    return;
  }
  TO* c = (TO*)p.C + zo * p.sc_o + zi * p.sc_i + m * p.ldc + n0;
  if (cnt == 4 && p.vec_store) {
    if (sizeof(TO) == 4) {
      gstore_f4(reinterpret_cast<float*>(c), *reinterpret_cast<const float(*)[4]>(v));
    } else {
      uint2 w;
      w.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
      w.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
      gstore8(c, w);
    }
  } else {
    for (int e = 0; e < cnt; ++e) gstore_elem(c + e, v[e]);
  }
}

// The kernel's only argument is a GemmParams by value, at offset 0 of the kernarg segment.
// The epilogue re-reads it through an opaque copy of the segment pointer: those loads
// cannot be hoisted to the kernel entry, so the ~40 scalar registers of epilogue fields
// are not held across the K loop (holding them made the large tiles spill to scratch).
typedef __attribute__((address_space(4))) const uint32_t ConstU32;
__device__ __forceinline__ GemmParams late_params() {
  static_assert(sizeof(GemmParams) % 4 == 0, "GemmParams must be whole dwords");
  ConstU32* src = (ConstU32*)__builtin_amdgcn_kernarg_segment_ptr();
  asm volatile("" : "+s"(src));
  GemmParams e;
  uint32_t* dst = reinterpret_cast<uint32_t*>(&e);
#pragma unroll
  for (int i = 0; i < (int)(sizeof(GemmParams) / 4); ++i) dst[i] = src[i];
  return e;
}

// Epilogue of an MFMA accumulator block: acc[i][j] holds rows mb + 16 i and columns
// nb + 16 j .. +3 of this lane. Bias is loaded once per column fragment, 64-bit row
// addresses once per row, and the head scatter splits rows (batch, time) and columns
// (part, head, d) with one fast division each.
template <typename TO, int TM, int TN>
__device__ __forceinline__ void mfma_epilogue(const GemmParams& e, int64_t zo, int64_t zi,
                                              int64_t mb, int64_t nb, f32x4 (&acc)[TM][TN]) {
  int cnt[TN];
  float bias[TN][4];
#pragma unroll
  for (int j = 0; j < TN; ++j) {
    const int64_t n = nb + 16 * j;
    cnt[j] = n >= e.N ? 0 : (e.N - n >= 4 ? 4 : (int)(e.N - n));
  }
  // one branch around all the bias loads (a branch per load would wait inside each)
  if (e.bias) {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) bias[j][q] = bias_at(e, nb + 16 * j + q);
  } else {
#pragma unroll
    for (int j = 0; j < TN; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q) bias[j][q] = 0.f;
  }
  auto finish = [&](float (&v)[4], int j) {
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      if (e.divisor != 1.0f) v[q] = v[q] / e.divisor;
      v[q] = v[q] + bias[j][q];
      if (e.act != TL_ACT_NONE && !e.geglu) v[q] = apply_act(v[q], e.act);
    }
  };
  if (e.qkv) {
    // column split, once per fragment: part (Q, K or V), head h, offset d
    const int qw = e.Hq * e.Dh, kw = e.Hkv * e.Dh;
    TO* cbase[TN];
    int part[TN];
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int n = (int)(nb + 16 * j);
      part[j] = n < qw ? 0 : (n < qw + kw ? 1 : 2);
      const int nn = n - (part[j] == 0 ? 0 : (part[j] == 1 ? qw : qw + kw));
      const int h = (int)fast_div((uint32_t)nn, e.div_Dh), d = nn - h * e.Dh;
      cbase[j] = part[j] == 0 ? (TO*)e.q + ((int64_t)h * e.T) * e.Dh + d
               : part[j] == 1 ? (TO*)e.k + ((int64_t)h * e.L) * e.Dh + d
                              : (TO*)e.vt + ((int64_t)h * e.Dh + d) * e.L;
    }
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t m = mb + 16 * i;
      if (m >= e.M) continue;
      const int b = (int)fast_div((uint32_t)m, e.div_T), t = (int)m - b * e.T;
      const int pos0 = e.pos0_dev ? (int)*e.pos0_dev : e.pos0;
      const bool in_cache = t + pos0 < e.L;  // a device position past the cache: no K/V rows
      const int64_t rq = ((int64_t)b * e.Hq * e.T + t) * e.Dh;
      const int64_t rk = ((int64_t)b * e.Hkv * e.L + t + pos0) * e.Dh;
      const int64_t rv = (int64_t)b * e.Hkv * e.Dh * e.L + t + pos0;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if (cnt[j] == 0) continue;
        float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        finish(v, j);
        if (part[j] > 0 && !in_cache) continue;
        if (part[j] < 2) {
          TO* dst = cbase[j] + (part[j] == 0 ? rq : rk);
          if (sizeof(TO) == 2) {
            uint2 w;
            w.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
            w.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
            gstore8(dst, w);
          } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) gstore_elem(dst + q, v[q]);
          }
        } else {
          TO* dst = cbase[j] + rv;
#pragma unroll
          for (int q = 0; q < 4; ++q) gstore_elem(dst + (int64_t)q * e.L, v[q]);
        }
      }
    }
    return;
  }
  TO* cz = (TO*)e.C + zo * e.sc_o + zi * e.sc_i;
  if (e.geglu) {  // columns (gate f, up f, gate f+1, up f+1) with f = n / 2
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int64_t m = mb + 16 * i;
      if (m >= e.M) continue;
      TO* crow = cz + m * e.ldc + nb / 2;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        if (cnt[j] == 0) continue;
        float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        finish(v, j);
        const float h0 = apply_act(v[0], e.act) * v[1], h1 = apply_act(v[2], e.act) * v[3];
        TO* c = crow + 8 * j;
        if (sizeof(TO) == 2 && cnt[j] == 4 && e.vec_store) {
          gstore(reinterpret_cast<uint32_t*>(c), (uint32_t)f2bf(h0) | ((uint32_t)f2bf(h1) << 16));
        } else {
          gstore_elem(c, h0);
          if (cnt[j] == 4) gstore_elem(c + 1, h1);
        }
      }
    }
    return;
  }
  const TO* rz = e.res ? (const TO*)e.res + zo * e.sr_o + zi * e.sr_i : nullptr;
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int64_t m = mb + 16 * i;
    // the row's vector residual pieces, requested together before any is used (reads of
    // rows past M or of fragments that end past N are clamped in bounds and not used)
    float rq[TN][4];
    if (rz && e.vec_res) {
      const TO* r0 = rz + (m < e.M ? m : e.M - 1) * e.ldr;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t c = nb + 16 * j;
        const TO* src = r0 + (c + 4 <= e.N ? c : 0);
        if constexpr (sizeof(TO) == 2) {
          const uint2 u = gload8(src);
          rq[j][0] = __uint_as_float(u.x << 16); rq[j][1] = __uint_as_float(u.x & 0xffff0000u);
          rq[j][2] = __uint_as_float(u.y << 16); rq[j][3] = __uint_as_float(u.y & 0xffff0000u);
        } else {
          gload_f4(reinterpret_cast<const float*>(src), rq[j]);
        }
      }
    }
    if (m >= e.M) continue;
    TO* crow = cz + m * e.ldc + nb;
    const TO* rrow = rz ? rz + m * e.ldr + nb : nullptr;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      if (cnt[j] == 0) continue;
      float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      finish(v, j);
      if (rrow) {
        if (cnt[j] == 4 && e.vec_res) {
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = v[q] + rq[j][q];
        } else {
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (q < cnt[j]) v[q] = v[q] + gload_elem(rrow + 16 * j + q);
        }
      }
      TO* c = crow + 16 * j;
      if (cnt[j] == 4 && e.vec_store) {
        if (sizeof(TO) == 4) {
          gstore_f4(reinterpret_cast<float*>(c), v);
        } else {
          uint2 w;
          w.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
          w.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
          gstore8(c, w);
        }
      } else {
        for (int q = 0; q < cnt[j]; ++q) gstore_elem(c + q, v[q]);
      }
    }
  }
}

// Position i of the grouped tile order -> output tile (tm, tn): groups of group_m
// tile-rows, walked row-fastest.
__device__ __forceinline__ void grouped_tile(int i, const GemmParams& p, int& tm, int& tn) {
  const int per_group = p.group_m * p.tiles_n;
  const int g = i / per_group;
  const int first_m = g * p.group_m;
  const int gm = min(p.tiles_m - first_m, p.group_m);
  const int k = i - g * per_group;
  tm = first_m + k % gm;
  tn = k / gm;
}

// bf16 epilogue through LDS. Each wave applies its epilogue kind to its WM x WN results in
// fp32 (bias, then activation, then residual, as mfma_epilogue does), rounds them once to
// bf16 and writes them to its own LDS region; it then reads them back as 16-byte row pieces
// (U = WN / 8 per row), so each global store instruction writes whole row segments of
// 64 / U rows instead of 32-byte pieces of 16 rows (4x fewer cache lines touched per byte:
// the store issue time per tile drops about 4x). Piece u of row r sits at slot (u + r) % U,
// which spreads the fragment writes over the LDS banks. Only this wave touches its region
// and the LDS operations of one wave complete in order, so the reads need no barrier.
template <int KIND>
struct EpiTraits {
  static constexpr bool BIAS = KIND == EPI_BIAS || KIND == EPI_BIAS_GELU || KIND == EPI_BIAS_SILU ||
                               KIND == EPI_BIAS_RES;
  static constexpr bool RES = KIND == EPI_BIAS_RES || KIND == EPI_RES;
};

// The bias values of a lane's fragment columns nw + 16 j + 4 (lane / 16) + q (0 past N).
template <int KIND, int TN>
__device__ __forceinline__ void load_epi_bias(const GemmParams& e, int64_t nw,
                                              float (&bias)[EpiTraits<KIND>::BIAS ? TN : 1][4]) {
  if constexpr (EpiTraits<KIND>::BIAS) {
    const int fc = (threadIdx.x & 63) >> 4;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t n = nw + 16 * j + 4 * fc;
#pragma unroll
      for (int q = 0; q < 4; ++q) bias[j][q] = bias_at(e, n + q);
    }
  }
}

// Applies epilogue KIND to the fragment rows i = I0 .. I0 + NI - 1 of a wave's accumulators
// (block rows 16 I0 .. 16 (I0 + NI) - 1, starting at global row mw + 16 I0) and writes them,
// rounded once to bf16, to the region as 16-byte row pieces: piece u of staged row r at slot
// (r * U + (u + r) % U), U = WN / 8 (the rotation spreads the fragment writes over the LDS
// banks).
template <int KIND, int TM, int TN, int WN, int I0, int NI>
__device__ __forceinline__ void stage_rows(const GemmParams& e, const bf16_t* rz, int64_t mw,
                                           int64_t nw, f32x4 (&acc)[TM][TN],
                                           const float (&bias)[EpiTraits<KIND>::BIAS ? TN : 1][4],
                                           uint8_t* reg) {
  constexpr bool BIAS = EpiTraits<KIND>::BIAS, RES = EpiTraits<KIND>::RES;
  constexpr int U = WN / 8;
  const int lane = threadIdx.x & 63, fr = lane & 15, fc = lane >> 4;
  // All residual pieces of these rows are requested before any is used (one memory round
  // trip, not one per fragment). Rows past M and columns past N are computed and staged but
  // never stored, so their reads are clamped to the last row and to column N - 4 (N % 4 == 0
  // on this path) and their values do not matter.
  uint2 rv[RES ? NI : 1][RES ? TN : 1];
  if constexpr (RES) {
#pragma unroll
    for (int ii = 0; ii < NI; ++ii) {
      const int64_t m = mw + 16 * (I0 + ii) + fr;
      const bf16_t* rrow = rz + (m < e.M ? m : e.M - 1) * e.ldr;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int64_t n = nw + 16 * j + 4 * fc;
        rv[ii][j] = gload8(rrow + (n < e.N ? n : e.N - 4));
      }
    }
  }
#pragma unroll
  for (int ii = 0; ii < NI; ++ii) {
    const int i = I0 + ii, r = 16 * ii + fr;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      if (BIAS) {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = v[q] + bias[BIAS ? j : 0][q];
      }
      if (KIND == EPI_BIAS_GELU) {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = gelu_tanh(v[q]);
      }
      if (KIND == EPI_BIAS_SILU) {
#pragma unroll
        for (int q = 0; q < 4; ++q) v[q] = silu_tanh(v[q]);
      }
      if constexpr (RES) {
        const uint2 w = rv[ii][j];
        v[0] = v[0] + __uint_as_float(w.x << 16);
        v[1] = v[1] + __uint_as_float(w.x & 0xffff0000u);
        v[2] = v[2] + __uint_as_float(w.y << 16);
        v[3] = v[3] + __uint_as_float(w.y & 0xffff0000u);
      }
      uint2 w;
      w.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
      w.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
      const int u = 2 * j + (fc >> 1);
      *reinterpret_cast<uint2*>(reg + (r * U + (u + r) % U) * 16 + (fc & 1) * 8) = w;
    }
  }
}

// bf16 epilogue through LDS. Each wave applies its epilogue kind to its WM x WN results in
// fp32 (bias, then activation, then residual, as mfma_epilogue does), stages them in its own
// LDS region (stage_rows) and reads them back as 16-byte row pieces, so each global store
// instruction writes whole row segments of 64 / U rows instead of 32-byte pieces of 16 rows
// (4x fewer cache lines touched per byte: the store issue time per tile drops about 4x).
// Only this wave touches its region and the LDS operations of one wave complete in order,
// so the reads need no barrier.
template <int KIND, int TM, int TN, int WM, int WN>
__device__ __forceinline__ void staged_epilogue(const GemmParams& e, int64_t zo, int64_t zi,
                                                int64_t mw, int64_t nw, f32x4 (&acc)[TM][TN],
                                                bf16_t* region) {
  constexpr int U = WN / 8;
  static_assert(WN % 16 == 0 && (WM * U) % 64 == 0, "staged epilogue shape");
  const int lane = threadIdx.x & 63;
  uint8_t* reg = reinterpret_cast<uint8_t*>(region);
  float bias[EpiTraits<KIND>::BIAS ? TN : 1][4];
  load_epi_bias<KIND, TN>(e, nw, bias);
  const bf16_t* rz = EpiTraits<KIND>::RES ? (const bf16_t*)e.res + zo * e.sr_o + zi * e.sr_i : nullptr;
  stage_rows<KIND, TM, TN, WN, 0, TM>(e, rz, mw, nw, acc, bias, reg);
  bf16_t* cz = (bf16_t*)e.C + zo * e.sc_o + zi * e.sc_i;
#pragma unroll
  for (int p = 0; p < WM * U / 64; ++p) {
    const int q = p * 64 + lane, r = q / U, u = q - r * U;
    const uint4 val = *reinterpret_cast<const uint4*>(reg + (r * U + (u + r) % U) * 16);
    const int64_t m = mw + r, n = nw + 8 * u;
    if (m >= e.M || n >= e.N) continue;
    bf16_t* c = cz + m * e.ldc + n;
    if (n + 8 <= e.N) {
      gstore16(c, val);
    } else {  // the row's last piece when N % 8 != 0
      const uint32_t h[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
      for (int t = 0; t < 8; ++t)
        if (n + t < e.N) gstore(c + t, (bf16_t)(h[t >> 1] >> (16 * (t & 1))));
    }
  }
}

// QKV head scatter through LDS (bf16, D a multiple of 8). A wave whose column slab lies in Q
// or K stages its rows as above and writes each 16-byte row piece (8 consecutive d of one
// head) to q[b, h, t, :] or k[b, h, pos0 + t, :]. A slab in V is staged transposed (column c
// holds the WM rows, its 16-byte units rotated by c against bank conflicts) and each unit,
// 8 consecutive rows of one d, goes to vt[b, h, d, pos0 + t .. + 7]: as one 16-byte store
// when T, the cache capacity L and pos0 are multiples of 8 (the 8 rows then share b and the
// destination is aligned), or, with VELEM (any T, L and pos0; ViT-S/4: T = 65), as 8
// 2-byte stores with a (b, t) per row, which still writes runs of consecutive t. Returns
// false (nothing written) for a slab that straddles two parts; the caller then runs the
// generic epilogue for that wave.
template <bool BIAS, int TM, int TN, int WM, int WN, bool VELEM = false>
__device__ __forceinline__ bool staged_qkv_epilogue(const GemmParams& e, int64_t mw, int64_t nw,
                                                    f32x4 (&acc)[TM][TN], bf16_t* region) {
  constexpr int U = WN / 8, RU = WM / 8;
  static_assert(WN % 16 == 0 && (WM * U) % 64 == 0 && WM % 8 == 0, "staged qkv shape");
  const int qw = e.Hq * e.Dh, kw = e.Hkv * e.Dh;
  if (nw >= e.N) return true;  // slab past N: nothing to write
  const int n_lo = (int)nw, n_hi = (int)min(nw + WN, e.N) - 1;
  const int part = n_lo < qw ? 0 : (n_lo < qw + kw ? 1 : 2);
  const int part_hi = n_hi < qw ? 0 : (n_hi < qw + kw ? 1 : 2);
  if (part_hi != part) return false;
  const int lane = threadIdx.x & 63, fr = lane & 15, fc = lane >> 4;
  uint8_t* reg = reinterpret_cast<uint8_t*>(region);
  float bias[BIAS ? TN : 1][4];
  if (BIAS) {
#pragma unroll
    for (int j = 0; j < (BIAS ? TN : 1); ++j) {
      const int64_t n = nw + 16 * j + 4 * fc;
#pragma unroll
      for (int q = 0; q < 4; ++q) bias[j][q] = bias_at(e, n + q);
    }
  }
  const int base = part == 0 ? 0 : (part == 1 ? qw : qw + kw);
  if (part < 2) {
    // destination of this part, selected once: q [B, Hq, T, D] or k [B, Hkv, L, D] at pos0
    const uintptr_t dbase = part == 0 ? (uintptr_t)e.q : (uintptr_t)e.k;
    const int heads = part == 0 ? e.Hq : e.Hkv, tdim = part == 0 ? e.T : e.L;
    const int toff = part == 0 ? 0 : e.pos0;
#pragma unroll
    for (int i = 0; i < TM; ++i) {
      const int r = 16 * i + fr;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
        if (BIAS) {
#pragma unroll
          for (int q = 0; q < 4; ++q) v[q] = v[q] + bias[BIAS ? j : 0][q];
        }
        uint2 w;
        w.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
        w.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
        const int u = 2 * j + (fc >> 1);
        *reinterpret_cast<uint2*>(reg + (r * U + (u + r) % U) * 16 + (fc & 1) * 8) = w;
      }
    }
#pragma unroll
    for (int p = 0; p < WM * U / 64; ++p) {
      const int q = p * 64 + lane, r = q / U, u = q - r * U;
      const uint4 val = *reinterpret_cast<const uint4*>(reg + (r * U + (u + r) % U) * 16);
      const int64_t m = mw + r, n = nw + 8 * u;
      if (m >= e.M || n >= e.N) continue;
      const int b = (int)fast_div((uint32_t)m, e.div_T), t = (int)m - b * e.T;
      const int nn = (int)n - base;
      const int h = (int)fast_div((uint32_t)nn, e.div_Dh), d = nn - h * e.Dh;
      gstore16(reinterpret_cast<bf16_t*>(dbase) + ((int64_t)(b * heads + h) * tdim + t + toff) * e.Dh + d, val);
    }
    return true;
  }
  // V: transposed staging, element (column c, row r) at column c's unit (r / 8 + c) % RU
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int r = 16 * i + fr;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float v = acc[i][j][q];
        if (BIAS) v = v + bias[BIAS ? j : 0][q];
        const int c = 16 * j + 4 * fc + q;
        *reinterpret_cast<bf16_t*>(reg + (c * RU + ((r >> 3) + c) % RU) * 16 + (r & 7) * 2) = f2bf(v);
      }
    }
  }
#pragma unroll
  for (int p = 0; p < WN * RU / 64; ++p) {
    const int q = p * 64 + lane, c = q / RU, ru = q - c * RU;
    const uint4 val = *reinterpret_cast<const uint4*>(reg + (c * RU + (ru + c) % RU) * 16);
    const int64_t m = mw + 8 * ru, n = nw + c;
    if (m >= e.M || n >= e.N) continue;
    if constexpr (!VELEM) {  // rows m .. m+7 share b and start an aligned run of 8 positions
      const int b = (int)fast_div((uint32_t)m, e.div_T), t = (int)m - b * e.T;
      const int nn = (int)n - base;
      const int h = (int)fast_div((uint32_t)nn, e.div_Dh), d = nn - h * e.Dh;
      gstore16((bf16_t*)e.vt + ((int64_t)(b * e.Hkv + h) * e.Dh + d) * e.L + t + e.pos0, val);
    } else {
      const int nn = (int)n - base;
      const int h = (int)fast_div((uint32_t)nn, e.div_Dh), d = nn - h * e.Dh;
      const uint32_t hw[4] = {val.x, val.y, val.z, val.w};
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        const int64_t mj = m + j;
        if (mj >= e.M) break;
        const int b = (int)fast_div((uint32_t)mj, e.div_T), t = (int)mj - b * e.T;
        gstore((bf16_t*)e.vt + ((int64_t)(b * e.Hkv + h) * e.Dh + d) * e.L + t + e.pos0,
               (bf16_t)(hw[j >> 1] >> (16 * (j & 1))));
      }
    }
  }
  return true;
}

// Gated (GeGLU) epilogue through LDS: columns come in (gate f, up f) pairs, so a lane's 4
// results give 2 outputs act(gate) * up; the wave's WN / 2 output columns are staged as
// packed pairs and written as 16-byte row pieces (bf16, no bias, N / 2 % 8 == 0).
template <int KIND, int TM, int TN, int WM, int WN>
__device__ __forceinline__ void staged_geglu_epilogue(const GemmParams& e, int64_t zo, int64_t zi,
                                                      int64_t mw, int64_t nw,
                                                      f32x4 (&acc)[TM][TN], bf16_t* region) {
  constexpr int U = WN / 16;  // 16-byte output pieces per row (8 outputs each)
  static_assert(WN % 16 == 0 && (WM * U) % 64 == 0, "staged gated shape");
  const int lane = threadIdx.x & 63, fr = lane & 15, fc = lane >> 4;
  uint8_t* reg = reinterpret_cast<uint8_t*>(region);
#pragma unroll
  for (int i = 0; i < TM; ++i) {
    const int r = 16 * i + fr;
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const f32x4 v = acc[i][j];
      const float h0 = (KIND == EPI_GEGLU_GELU ? gelu_tanh(v[0]) : silu_tanh(v[0])) * v[1];
      const float h1 = (KIND == EPI_GEGLU_GELU ? gelu_tanh(v[2]) : silu_tanh(v[2])) * v[3];
      // output columns 8 j + 2 fc, +1 of this wave: piece j, bytes 4 fc
      *reinterpret_cast<uint32_t*>(reg + (r * U + (j + r) % U) * 16 + 4 * fc) =
          (uint32_t)f2bf(h0) | ((uint32_t)f2bf(h1) << 16);
    }
  }
  bf16_t* cz = (bf16_t*)e.C + zo * e.sc_o + zi * e.sc_i;
  const int64_t nout = e.N / 2, ow = nw / 2;
#pragma unroll
  for (int p = 0; p < WM * U / 64; ++p) {
    const int q = p * 64 + lane, r = q / U, u = q - r * U;
    const uint4 val = *reinterpret_cast<const uint4*>(reg + (r * U + (u + r) % U) * 16);
    const int64_t m = mw + r, n = ow + 8 * u;
    if (m >= e.M || n >= nout) continue;
    gstore16(cz + m * e.ldc + n, val);
  }
}

// Block id -> output tile: workgroups are dispatched round-robin over the 8 XCDs, so XCD x
// runs blocks x, x+8, ...; give it the contiguous run [x q + min(x, r), ...) of the
// grouped order.
__device__ __forceinline__ void map_tile(int bid, const GemmParams& p, int& tm, int& tn) {
  const int ntiles = p.tiles_m * p.tiles_n;
  const int x = bid & 7, local = bid >> 3;
  const int q = ntiles >> 3, r = ntiles & 7;
  grouped_tile(x * q + min(x, r) + local, p, tm, tn);
}

template <typename TO, int BM, int BN, int WGM, int WGN>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_mfma_kernel(GemmParams p) {
  constexpr int NT = 64 * WGM * WGN;       // WGM x WGN waves
  constexpr int BK = 64;                   // bf16 elements of K per step: 8 chunks of 16 B
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int RPP = NT / 8;              // tile rows one load pass covers (8 chunks per row)
  constexpr int A_CH = BM / RPP, B_CH = BN / RPP;
  static_assert(BM % RPP == 0 && BN % RPP == 0 && RPP % 8 == 0, "bad tile/thread split");
  static_assert(TM >= 1 && TN >= 1, "wave tile below one MFMA tile");
  __shared__ __attribute__((aligned(16))) bf16_t As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][BN * BK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave - wm * WGN;
  const int64_t z = blockIdx.z;
  const int64_t zo = z / p.batch_inner, zi = z - zo * p.batch_inner;
  int tm, tn;
  map_tile(blockIdx.x, p, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t K = p.K;

  // Uniform tile bases plus 32-bit per-pass element offsets (rows past M or N are clamped
  // to the last row: computed, never stored). Every pass shares one LDS swizzle slot
  // because RPP is a multiple of 8.
  const bf16_t* Ab = (const bf16_t*)p.A + zo * p.sa_o + zi * p.sa_i + m0 * p.lda;
  const bf16_t* Bb = (const bf16_t*)p.B + zo * p.sb_o + zi * p.sb_i + n0 * p.ldb;
  const int lr = tid >> 3, lc = tid & 7;
  const int slot = lr * BK + ((lc ^ (lr & 7)) << 3);
  uint32_t a_off[A_CH], b_off[B_CH];
  {
    const int a_last = (int)min((int64_t)BM - 1, p.M - 1 - m0);
    const int b_last = (int)min((int64_t)BN - 1, p.N - 1 - n0);
#pragma unroll
    for (int i = 0; i < A_CH; ++i) a_off[i] = (uint32_t)(min(i * RPP + lr, a_last) * p.lda + lc * 8);
#pragma unroll
    for (int i = 0; i < B_CH; ++i) b_off[i] = (uint32_t)(min(i * RPP + lr, b_last) * p.ldb + lc * 8);
  }
  uint4 ra[A_CH], rb[B_CH];
  auto load_tile = [&](int64_t k0) {
    const bf16_t* a = Ab + k0;
    const bf16_t* b = Bb + k0;
    if (k0 + BK <= K) {
#pragma unroll
      for (int i = 0; i < A_CH; ++i) ra[i] = *reinterpret_cast<const uint4*>(a + a_off[i]);
#pragma unroll
      for (int i = 0; i < B_CH; ++i) rb[i] = *reinterpret_cast<const uint4*>(b + b_off[i]);
    } else {  // K tail: K % 8 == 0, so a chunk is either fully inside K or fully outside
      const bool in = k0 + lc * 8 < K;
#pragma unroll
      for (int i = 0; i < A_CH; ++i)
        ra[i] = in ? *reinterpret_cast<const uint4*>(a + a_off[i]) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < B_CH; ++i)
        rb[i] = in ? *reinterpret_cast<const uint4*>(b + b_off[i]) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) *reinterpret_cast<uint4*>(&As[buf][slot + i * RPP * BK]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) *reinterpret_cast<uint4*>(&Bs[buf][slot + i * RPP * BK]) = rb[i];
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)((K + BK - 1) / BK);
  load_tile(0);
  store_tile(0);
  __syncthreads();
  const int fr = lane & 15, fc = lane >> 4;
  // fragment rows are fr + multiples of 16, so their swizzle depends on fr only
  const int a_frag = (wm * WM + fr) * BK, b_frag = (wn * WN + fr) * BK;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tile((int64_t)(kt + 1) * BK);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int sw = ((s * 4 + fc) ^ (fr & 7)) << 3;
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&As[cur][a_frag + i * 16 * BK + sw]);
#pragma unroll
      for (int j = 0; j < TN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(&Bs[cur][b_frag + j * 16 * BK + sw]);
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tile(cur ^ 1);
    __syncthreads();
  }

  const GemmParams e = late_params();
  mfma_epilogue<TO, TM, TN>(e, zo, zi, m0 + wm * WM + fr, n0 + wn * WN + 4 * fc, acc);
}

// gemm_mfma_f32_kernel: fp32 operands on the matrix cores (v_mfma_f32_16x16x4f32: fp32
// products, fp32 accumulation), for the fp32 models (the reference's default FLOAT_TYPE).
// The gemm_mfma_kernel scheme with 4-byte elements: A [M, K] and B [N, K] both K-contiguous
// (K % 4 == 0, rows 16-byte aligned), 32-element K steps as 8 chunks of 16 B per row,
// XOR-swizzled in LDS, double-buffered through registers. A lane's 16-byte fragment feeds
// four MFMAs: MFMA q takes element q of every lane's chunk, so the four lane groups supply
// K indices 4c + q of their chunks c; A and B use the same assignment, which covers each K
// index of the step once. B is the first MFMA operand, so a lane's four results are four
// consecutive output columns of one row, the layout epilogue4 stores.
template <typename TO, int BM, int BN, int WGM, int WGN, int BK = 32>
__global__ __launch_bounds__(64 * WGM * WGN) void gemm_mfma_f32_kernel(GemmParams p) {
  constexpr int NT = 64 * WGM * WGN;
  constexpr int CPR = BK / 4;              // 16-byte chunks per row of a K step (8 or 4)
  constexpr int WM = BM / WGM, WN = BN / WGN;
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int RPP = NT / CPR;            // tile rows one load pass covers
  constexpr int A_CH = BM / RPP, B_CH = BN / RPP;
  static_assert(BK == 32 || BK == 16, "K step of 16 or 32 fp32 elements");
  static_assert(BM % RPP == 0 && BN % RPP == 0 && RPP % CPR == 0, "bad tile/thread split");
  static_assert(TM >= 1 && TN >= 1, "wave tile below one MFMA tile");
  __shared__ __attribute__((aligned(16))) float As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN * BK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave / WGN, wn = wave - wm * WGN;
  const int64_t z = blockIdx.z;
  const int64_t zo = z / p.batch_inner, zi = z - zo * p.batch_inner;
  int tm, tn;
  map_tile(blockIdx.x, p, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const int64_t K = p.K;

  const float* Ab = (const float*)p.A + zo * p.sa_o + zi * p.sa_i + m0 * p.lda;
  const float* Bb = (const float*)p.B + zo * p.sb_o + zi * p.sb_i + n0 * p.ldb;
  const int lr = tid / CPR, lc = tid % CPR;
  const int slot = lr * BK + ((lc ^ (lr & (CPR - 1))) << 2);
  uint32_t a_off[A_CH], b_off[B_CH];
  {
    // rows past M or N are clamped to the last row: computed, never stored
    const int a_last = (int)min((int64_t)BM - 1, p.M - 1 - m0);
    const int b_last = (int)min((int64_t)BN - 1, p.N - 1 - n0);
#pragma unroll
    for (int i = 0; i < A_CH; ++i) a_off[i] = (uint32_t)(min(i * RPP + lr, a_last) * p.lda + lc * 4);
#pragma unroll
    for (int i = 0; i < B_CH; ++i) b_off[i] = (uint32_t)(min(i * RPP + lr, b_last) * p.ldb + lc * 4);
  }
  uint4 ra[A_CH], rb[B_CH];
  auto load_tile = [&](int64_t k0) {
    const float* a = Ab + k0;
    const float* b = Bb + k0;
    if (k0 + BK <= K) {
#pragma unroll
      for (int i = 0; i < A_CH; ++i) ra[i] = *reinterpret_cast<const uint4*>(a + a_off[i]);
#pragma unroll
      for (int i = 0; i < B_CH; ++i) rb[i] = *reinterpret_cast<const uint4*>(b + b_off[i]);
    } else {  // K tail: K % 4 == 0, so a chunk is either fully inside K or fully outside
      const bool in = k0 + lc * 4 < K;
#pragma unroll
      for (int i = 0; i < A_CH; ++i)
        ra[i] = in ? *reinterpret_cast<const uint4*>(a + a_off[i]) : make_uint4(0, 0, 0, 0);
#pragma unroll
      for (int i = 0; i < B_CH; ++i)
        rb[i] = in ? *reinterpret_cast<const uint4*>(b + b_off[i]) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) *reinterpret_cast<uint4*>(&As[buf][slot + i * RPP * BK]) = ra[i];
#pragma unroll
    for (int i = 0; i < B_CH; ++i) *reinterpret_cast<uint4*>(&Bs[buf][slot + i * RPP * BK]) = rb[i];
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  const int nk = (int)((K + BK - 1) / BK);
  load_tile(0);
  store_tile(0);
  __syncthreads();
  const int fr = lane & 15, fc = lane >> 4;
  const int a_frag = (wm * WM + fr) * BK, b_frag = (wn * WN + fr) * BK;
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tile((int64_t)(kt + 1) * BK);
#pragma unroll
    for (int s = 0; s < BK / 16; ++s) {
      const int sw = ((s * 4 + fc) ^ (fr & (CPR - 1))) << 2;
      f32x4 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) af[i] = *reinterpret_cast<const f32x4*>(&As[cur][a_frag + i * 16 * BK + sw]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[j] = *reinterpret_cast<const f32x4*>(&Bs[cur][b_frag + j * 16 * BK + sw]);
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int i = 0; i < TM; ++i)
#pragma unroll
          for (int j = 0; j < TN; ++j)
            acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(bfr[j][q], af[i][q], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tile(cur ^ 1);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      epilogue4<float, TO>(p, zo, zi, m0 + wm * WM + fr + 16 * i, n0 + wn * WN + 16 * j + 4 * fc, v);
    }
}

// gemm_dma_kernel: same tiling and epilogue as gemm_mfma_kernel, for K % 64 == 0. Operand
// tiles move from global memory straight into LDS (global_load_lds_dwordx4: each lane of a
// wave writes its 16 bytes at LDS base + 16 * lane), so the pipeline can run STAGES - 1
// K steps ahead without holding any registers for them. Loaded memory latency on MI355X is
// a few K steps of MFMA work, which a one-step register prefetch cannot cover. Each stage
// is a separate LDS array and the K loop is unrolled over the stages, so the compiler's
// wait counters can tell the stage being read from the stages being filled. Before reading
// a stage a wave waits until only the later stages' loads are outstanding (vmcnt counts
// its own loads in issue order) and its LDS reads are done, then meets the other waves at
// a barrier. A load group is 8 tile rows x 8 chunks = 1 KB: lane l fills row l / 8, slot
// l % 8, which holds logical chunk (l % 8) ^ (row % 8), the XOR swizzle the fragment
// reads undo.
// Scheduling pattern for one K step of fragment reads and MFMAs: NR reads of the first
// half, then the second half's NR reads each followed by a share of the first half's NM
// MFMAs, then the second half's NM MFMAs. The fragment registers of both halves stay live,
// so no MFMA waits for an LDS read issued right before it.
template <int NR, int NM, int R = 0>
__device__ __forceinline__ void interleave_reads_mfma() {
  if constexpr (R < NR) {
    constexpr int q = NM / NR, rem = NM % NR;
    __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);                       // DS read
    __builtin_amdgcn_sched_group_barrier(0x008, q + (R < rem ? 1 : 0), 0);  // MFMA
    interleave_reads_mfma<NR, NM, R + 1>();
  }
}
template <int NR, int NM>
__device__ __forceinline__ void schedule_kstep() {
  __builtin_amdgcn_sched_group_barrier(0x100, NR, 0);
  interleave_reads_mfma<NR, NM>();
  __builtin_amdgcn_sched_group_barrier(0x008, NM, 0);
}


template <typename TO, int BM, int BN, int WGM, int WGN, int WPE, int STAGES, bool VELEM = false>
__global__ __launch_bounds__(64 * WGM * WGN) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void gemm_dma_kernel(GemmParams p) {
  constexpr int NW = WGM * WGN, BK = 64;
  constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
  // 1 KB load groups per K step: GA of A, then GB of B. Waves 0..R-1 issue LMAX of them,
  // the others LMAX - 1 (when NW does not divide the count), each wave waiting on its own.
  constexpr int GA = BM / 8, GB = BN / 8, GT = GA + GB;
  constexpr int LMAX = (GT + NW - 1) / NW, R = GT - (LMAX - 1) * NW;
  static_assert(TM >= 1 && TN >= 1, "bad tile/wave split");
  static_assert(STAGES == 2 || STAGES == 3, "2 or 3 stages");
  static_assert(LMAX * (STAGES - 2) <= 63, "vmcnt range");
  constexpr int SZ = (BM + BN) * BK;
  __shared__ __attribute__((aligned(16))) bf16_t S0[SZ];
  __shared__ __attribute__((aligned(16))) bf16_t S1[SZ];
  __shared__ __attribute__((aligned(16))) bf16_t S2[STAGES > 2 ? SZ : 8];
  auto stage = [&](int i) -> bf16_t* { return i == 0 ? S0 : (i == 1 ? S1 : S2); };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave - wm * WGN;
  const bool full = wave < R;  // this wave issues LMAX groups per K step
  const int g0 = full ? wave * LMAX : R * LMAX + (wave - R) * (LMAX - 1);
  const int64_t z = blockIdx.z;
  const int64_t zo = z / p.batch_inner, zi = z - zo * p.batch_inner;
  int tm, tn;
  map_tile(blockIdx.x, p, tm, tn);
  const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * BN;
  const bf16_t* Ab = (const bf16_t*)p.A + zo * p.sa_o + zi * p.sa_i + m0 * p.lda;
  const bf16_t* Bb = (const bf16_t*)p.B + zo * p.sb_o + zi * p.sb_i + n0 * p.ldb;
  uint32_t off[LMAX];
  {
    const int a_last = (int)min((int64_t)BM - 1, p.M - 1 - m0);
    const int b_last = (int)min((int64_t)BN - 1, p.N - 1 - n0);
    const int rin = lane >> 3, c = (lane & 7) ^ rin;
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
      const int g = min(g0 + j, GT - 1);
      off[j] = g < GA ? (uint32_t)(min(8 * g + rin, a_last) * p.lda + c * 8)
                      : (uint32_t)(min(8 * (g - GA) + rin, b_last) * p.ldb + c * 8);
    }
  }
  auto issue = [&](bf16_t* S, int64_t k0) {
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
      if (j == LMAX - 1 && !full) break;
      const int g = g0 + j;
      const bf16_t* src = (g < GA ? Ab : Bb) + k0 + off[j];
      dma_load16(src, lds_offset(S + g * 512));
    }
  };
  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fr = lane & 15, fc = lane >> 4;
  const int a_frag = (wm * WM + fr) * BK, b_frag = BM * BK + (wn * WN + fr) * BK;
  // Both 32-wide K halves' fragments are read into their own registers; the second half's
  // reads are spread over the first half's MFMAs (schedule_kstep).
  auto compute = [&](const bf16_t* S) {
    bf16x8 af[2][TM], bfr[2][TN];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int swh = ((h * 4 + fc) ^ (fr & 7)) << 3;
#pragma unroll
      for (int i = 0; i < TM; ++i) af[h][i] = *reinterpret_cast<const bf16x8*>(&S[a_frag + i * 16 * BK + swh]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[h][j] = *reinterpret_cast<const bf16x8*>(&S[b_frag + j * 16 * BK + swh]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[h][j], af[h][i], acc[i][j], 0, 0, 0);
    schedule_kstep<TM + TN, TM * TN>();
  };
  const int nk = (int)(p.K / BK);
#pragma unroll
  for (int i = 0; i < STAGES - 1; ++i)
    if (i < nk) issue(stage(i), (int64_t)i * BK);
  for (int kt = 0; kt < nk; kt += STAGES) {
#pragma unroll
    for (int u = 0; u < STAGES; ++u) {
      const int t = kt + u;
      if (t >= nk) break;
      // tiles t+1 .. t+STAGES-2 may stay in flight
      if (STAGES == 3 && t + 1 < nk) {
        if (full) dma_stage_sync<LMAX * (STAGES - 2)>();
        else dma_stage_sync<(LMAX - 1) * (STAGES - 2)>();
      } else {
        dma_stage_sync<0>();
      }
      if (t + STAGES - 1 < nk) issue(stage((u + STAGES - 1) % STAGES), (int64_t)(t + STAGES - 1) * BK);
      compute(stage(u));
    }
  }

  const GemmParams e = late_params();
  bool done = false;
  if constexpr (sizeof(TO) == 2) {
    if (e.epi != EPI_GENERIC) {
      // each wave's WM x WN block goes to its own region of the stage arrays, once every
      // wave has finished reading the last stage
      constexpr int WPA = SZ / (WM * WN);  // wave regions per stage array
      static_assert(WPA >= 1 && (NW + WPA - 1) / WPA <= STAGES, "staging space");
      __syncthreads();
      bf16_t* region = stage(wave / WPA) + (wave % WPA) * (WM * WN);
      const int64_t mw = m0 + wm * WM, nw = n0 + wn * WN;
      done = true;
      switch (e.epi) {
        case EPI_PLAIN: staged_epilogue<EPI_PLAIN, TM, TN, WM, WN>(e, zo, zi, mw, nw, acc, region); break;
        case EPI_BIAS: staged_epilogue<EPI_BIAS, TM, TN, WM, WN>(e, zo, zi, mw, nw, acc, region); break;
        case EPI_BIAS_GELU: staged_epilogue<EPI_BIAS_GELU, TM, TN, WM, WN>(e, zo, zi, mw, nw, acc, region); break;
        case EPI_BIAS_SILU: staged_epilogue<EPI_BIAS_SILU, TM, TN, WM, WN>(e, zo, zi, mw, nw, acc, region); break;
        case EPI_BIAS_RES: staged_epilogue<EPI_BIAS_RES, TM, TN, WM, WN>(e, zo, zi, mw, nw, acc, region); break;
        case EPI_RES: staged_epilogue<EPI_RES, TM, TN, WM, WN>(e, zo, zi, mw, nw, acc, region); break;
        case EPI_QKV_BIAS: done = staged_qkv_epilogue<true, TM, TN, WM, WN, VELEM>(e, mw, nw, acc, region); break;
        case EPI_GEGLU_GELU: staged_geglu_epilogue<EPI_GEGLU_GELU, TM, TN, WM, WN>(e, zo, zi, mw, nw, acc, region); break;
        case EPI_GEGLU_SILU: staged_geglu_epilogue<EPI_GEGLU_SILU, TM, TN, WM, WN>(e, zo, zi, mw, nw, acc, region); break;
        default: done = staged_qkv_epilogue<false, TM, TN, WM, WN, VELEM>(e, mw, nw, acc, region); break;
      }
    }
  }
  // one call site: a wave whose QKV slab straddles two parts continues here
  if (!done) mfma_epilogue<TO, TM, TN>(e, zo, zi, m0 + wm * WM + fr, n0 + wn * WN + 4 * fc, acc);
}

// Stores of a persistent tile's staged rows through a buffer resource: a piece outside the
// M x N output gets offset 0x80000000, past the resource's num_records, and the hardware
// drops it. Every lane of every wave therefore issues the same number of store instructions
// per tile, which the K pipeline's wait counts rely on.
typedef __amdgpu_buffer_rsrc_t BufRsrc;
__device__ __forceinline__ BufRsrc make_c_rsrc(const GemmParams& e) {
  // raw buffer (stride 0); 0x00020000: the gfx9 data-format word for untyped dword access
  const uint32_t extent = (uint32_t)(((e.M - 1) * e.ldc + e.N) * 2);
  return __builtin_amdgcn_make_buffer_rsrc(e.C, (short)0, (int)extent, 0x00020000);
}

// gemm_dma_persistent_kernel: one workgroup per resident slot (gridDim.x = CUs x workgroups
// per CU, a multiple of 8), bf16 output with a staged epilogue kind (PLAIN .. RES), batch 1,
// N % 8 == 0 and an output extent below 2 GiB (host-checked). Workgroup b runs on XCD b % 8
// and walks that XCD's contiguous run of the grouped tile order with stride gridDim.x / 8,
// so the XCD's workgroups share A and B panels in its L2.
//
// Its K steps form one flattened pipeline across its tiles: the loads of the next tile's
// first STAGES - 1 steps are in flight while the current tile finishes, stages its epilogue
// in the LDS stage it has just consumed (in NH row groups when the tile is larger than one
// stage) and stores it. A short K loop (12 steps at K = 768) then pays the first-load latency
// once per workgroup, not once per tile.
//
// Wait counts: vmcnt counts the direct-to-LDS loads and the epilogue stores of a wave in
// issue order. Step t needs its own loads; issued after them are the next STAGES - 2 steps'
// loads (LMAX or LMAX - 1 per step for this wave) and the SPT stores of every tile that ended
// in steps t - STAGES + 1 .. t - 1. Bias and residual loads inside an epilogue are waited for
// before its stores, so they only make a wait stricter.
template <int KIND, int BM, int BN, int WGM, int WGN, int WPE, int STAGES>
__global__ __launch_bounds__(64 * WGM * WGN) __attribute__((amdgpu_waves_per_eu(WPE, WPE)))
void gemm_dma_persistent_kernel(GemmParams p) {
  constexpr int NW = WGM * WGN, BK = 64;
  constexpr int WM = BM / WGM, WN = BN / WGN, TM = WM / 16, TN = WN / 16;
  constexpr int GA = BM / 8, GB = BN / 8, GT = GA + GB;
  constexpr int LMAX = (GT + NW - 1) / NW, R = GT - (LMAX - 1) * NW;
  constexpr int SZ = (BM + BN) * BK;
  // row groups of the staged epilogue: NW regions of WM / NH rows x WN must fit one stage
  constexpr int NH = (BM * BN <= SZ) ? 1 : 2;
  constexpr int NI = TM / NH, U = WN / 8;
  constexpr int SPG = 16 * NI * U / 64;  // store instructions per wave per row group
  constexpr int SPT = NH * SPG;           // ... per tile
  static_assert(TM >= 1 && TN >= 1 && TM % NH == 0, "bad tile/wave split");
  static_assert(BM * BN <= NH * SZ && (16 * NI * U) % 64 == 0 && WN % 16 == 0, "epilogue staging");
  static_assert(STAGES == 2 || STAGES == 3, "2 or 3 stages");
  static_assert(LMAX * (STAGES - 2) + 2 * SPT <= 63, "vmcnt range");
  __shared__ __attribute__((aligned(16))) bf16_t S0[SZ];
  __shared__ __attribute__((aligned(16))) bf16_t S1[SZ];
  __shared__ __attribute__((aligned(16))) bf16_t S2[STAGES > 2 ? SZ : 8];
  auto stage = [&](int i) -> bf16_t* { return i == 0 ? S0 : (i == 1 ? S1 : S2); };

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WGN, wn = wave - wm * WGN;
  const bool full = wave < R;  // this wave issues LMAX groups per K step
  const int g0 = full ? wave * LMAX : R * LMAX + (wave - R) * (LMAX - 1);
  const int ntiles = p.tiles_m * p.tiles_n;
  const int bid = blockIdx.x, x = bid & 7, lb = bid >> 3, per_x = (int)gridDim.x >> 3;
  const int q8 = ntiles >> 3, r8 = ntiles & 7;
  const int cs = x * q8 + min(x, r8), cn = q8 + (x < r8 ? 1 : 0);
  const int my_tiles = lb < cn ? (cn - lb + per_x - 1) / per_x : 0;
  const int nk = (int)(p.K / BK);
  const int total = my_tiles * nk;
  auto tile_origin = [&](int rr, int64_t& m0, int64_t& n0) {
    int tm, tn;
    grouped_tile(cs + lb + rr * per_x, p, tm, tn);
    m0 = (int64_t)tm * BM;
    n0 = (int64_t)tn * BN;
  };

  // issue side: the tile and K step of the next load, its panel bases and row offsets
  int i_rr = 0, i_kk = 0;
  const bf16_t* iA = nullptr;
  const bf16_t* iB = nullptr;
  uint32_t off[LMAX];
  const int rin = lane >> 3, cch = (lane & 7) ^ rin;
  auto issue = [&](bf16_t* S) {
    if (i_kk == 0) {
      int64_t m0, n0;
      tile_origin(i_rr, m0, n0);
      iA = (const bf16_t*)p.A + m0 * p.lda;
      iB = (const bf16_t*)p.B + n0 * p.ldb;
      const int a_last = (int)min((int64_t)BM - 1, p.M - 1 - m0);
      const int b_last = (int)min((int64_t)BN - 1, p.N - 1 - n0);
#pragma unroll
      for (int j = 0; j < LMAX; ++j) {
        const int g = min(g0 + j, GT - 1);
        off[j] = g < GA ? (uint32_t)(min(8 * g + rin, a_last) * p.lda + cch * 8)
                        : (uint32_t)(min(8 * (g - GA) + rin, b_last) * p.ldb + cch * 8);
      }
    }
    const int64_t k0 = (int64_t)i_kk * BK;
#pragma unroll
    for (int j = 0; j < LMAX; ++j) {
      if (j == LMAX - 1 && !full) break;
      const int g = g0 + j;
      dma_load16((g < GA ? iA : iB) + k0 + off[j], lds_offset(S + g * 512));
    }
    if (++i_kk == nk) {
      i_kk = 0;
      ++i_rr;
    }
  };

  f32x4 acc[TM][TN];
#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  const int fr = lane & 15, fc = lane >> 4;
  const int a_frag = (wm * WM + fr) * BK, b_frag = BM * BK + (wn * WN + fr) * BK;
  auto compute = [&](const bf16_t* S) {
    bf16x8 af[2][TM], bfr[2][TN];
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int swh = ((h * 4 + fc) ^ (fr & 7)) << 3;
#pragma unroll
      for (int i = 0; i < TM; ++i) af[h][i] = *reinterpret_cast<const bf16x8*>(&S[a_frag + i * 16 * BK + swh]);
#pragma unroll
      for (int j = 0; j < TN; ++j) bfr[h][j] = *reinterpret_cast<const bf16x8*>(&S[b_frag + j * 16 * BK + swh]);
    }
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[h][j], af[h][i], acc[i][j], 0, 0, 0);
    schedule_kstep<TM + TN, TM * TN>();
  };

  // the staged epilogue of tile rr into stage S (every wave has finished reading S)
  auto finish_tile = [&](int rr, bf16_t* S) {
    int64_t m0, n0;
    tile_origin(rr, m0, n0);
    const GemmParams e = late_params();
    const int64_t mw = m0 + wm * WM, nw = n0 + wn * WN;
    const BufRsrc rs = make_c_rsrc(e);
    float bias[EpiTraits<KIND>::BIAS ? TN : 1][4];
    load_epi_bias<KIND, TN>(e, nw, bias);
    const bf16_t* rz = EpiTraits<KIND>::RES ? (const bf16_t*)e.res : nullptr;
    uint8_t* reg = reinterpret_cast<uint8_t*>(S + wave * (16 * NI * WN));
    auto write_group = [&](int i0) {
#pragma unroll
      for (int pc = 0; pc < SPG; ++pc) {
        const int qq = pc * 64 + lane, r = qq / U, u = qq - r * U;
        const uint4 v = *reinterpret_cast<const uint4*>(reg + (r * U + (u + r) % U) * 16);
        const int64_t m = mw + 16 * i0 + r, n = nw + 8 * u;
        const uint32_t o = (m < e.M && n < e.N) ? (uint32_t)((m * e.ldc + n) * 2) : 0x80000000u;
        const u32x4_t t = {v.x, v.y, v.z, v.w};
        __builtin_amdgcn_raw_buffer_store_b128(t, rs, (int)o, 0, 0);
      }
    };
    stage_rows<KIND, TM, TN, WN, 0, NI>(e, rz, mw, nw, acc, bias, reg);
    write_group(0);
    if constexpr (NH == 2) {
      stage_rows<KIND, TM, TN, WN, NI, NI>(e, rz, mw, nw, acc, bias, reg);
      write_group(NI);
    }
#pragma unroll
    for (int i = 0; i < TM; ++i)
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  };

#pragma unroll
  for (int i = 0; i < STAGES - 1; ++i)
    if (i < total) issue(stage(i));
  int c_rr = 0, c_kk = 0;  // compute side: tile and K step
  bool e1 = false, e2 = false;  // a tile ended at step t - 1 / t - 2
  for (int t0 = 0; t0 < total; t0 += STAGES) {
#pragma unroll
    for (int u = 0; u < STAGES; ++u) {
      const int t = t0 + u;
      if (t >= total) break;
      const int ends = (int)e1 + (int)(STAGES == 3 && e2);
      if (STAGES == 3 && t + 1 < total) {
        if (full) {
          if (ends == 0) dma_stage_sync<LMAX>();
          else if (ends == 1) dma_stage_sync<LMAX + SPT>();
          else dma_stage_sync<LMAX + 2 * SPT>();
        } else {
          if (ends == 0) dma_stage_sync<LMAX - 1>();
          else if (ends == 1) dma_stage_sync<LMAX - 1 + SPT>();
          else dma_stage_sync<LMAX - 1 + 2 * SPT>();
        }
      } else {
        if (ends == 0) dma_stage_sync<0>();
        else if (ends == 1) dma_stage_sync<SPT>();
        else dma_stage_sync<2 * SPT>();
      }
      if (t + STAGES - 1 < total) issue(stage((u + STAGES - 1) % STAGES));
      compute(stage(u));
      e2 = e1;
      e1 = ++c_kk == nk;
      if (e1) {
        // every wave has read stage u (a plain barrier: no wait on the loads in flight)
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
        finish_tile(c_rr, stage(u));
        c_kk = 0;
        ++c_rr;
      }
    }
  }
}

// gemm_skinny_kernel: M <= 16 (a decode step's few rows), where the product is a stream of
// the weights. A workgroup owns 16 rows of Bt (n0 .. n0 + 15) and its NW waves split K. Per
// 32-wide K step a wave loads one 16 x 32 fragment of Bt (lane: row lane % 16, 8 columns at
// 8 * (lane / 16), so the 4 lanes of a row read 64 contiguous bytes) and the matching A
// fragment (row m = lane % 16 of A, zeros for m >= M), and issues one MFMA with Bt as the
// first operand: lane holds out[m = lane % 16][n0 + 4 (lane / 16) + 0..3]. U steps are in
// flight per wave. The NW partial sums meet in LDS and the first wave runs the same
// epilogue as the fp32 kernel (bias, activation, residual, QKV scatter, gated pairs).
//
// With norm_rows set (NORM), each step also multiplies the A fragment by itself on the
// matrix cores (X X^T, one more MFMA per 32-wide step, no vector ALU work): its diagonal is
// each row's sum of squares, and the reduced sums are scaled by 1 / sqrt(mean + eps). With
// the norm's gain folded into B, that is RMSNorm(A) @ B without a separate pass over A.
// (Scaling the A fragments by the gain on the vector ALUs instead cost more than the norm's
// own launch: every workgroup repeats that work, 2048 times for the GeGLU product.)
//
// When there are too few 16-row blocks to fill the GPU, K is also split over gridDim.y
// workgroups: each writes its partial block (64 lanes x 4 floats) to `part`, and
// gemm_skinny_reduce_kernel, the next launch on the stream, sums them and runs the epilogue.
// (Letting the last-arriving workgroup reduce instead costs more than the launch it saves:
// publishing the partials across XCDs takes an agent-scope release and acquire, which on
// gfx950 write back and invalidate the whole L2 of the XCD, and the down projection of a
// config-5 decode step went from 18 to 31 us.)
template <typename TO, int NW, int U, bool NORM>
__global__ __launch_bounds__(64 * NW) void gemm_skinny_kernel(GemmParams p, float* part) {
  __shared__ f32x4 red[NW][64];
  __shared__ float ssq[NW][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int64_t z = blockIdx.z;
  const int64_t zo = z / p.batch_inner, zi = z - zo * p.batch_inner;
  const int64_t n0 = (int64_t)blockIdx.x * 16;
  const int64_t wrow = min(n0 + r, p.N - 1);
  const bf16_t* W = (const bf16_t*)p.B + zo * p.sb_o + zi * p.sb_i + wrow * p.ldb + 8 * g;
  const bool xrow = r < p.M;
  const bf16_t* X = (const bf16_t*)p.A + zo * p.sa_o + zi * p.sa_i +
                    (xrow ? r : 0) * p.lda + 8 * g;
  const int S = gridDim.y, ky = blockIdx.y;
  const int64_t nsteps = (p.K + 31) / 32;
  const int64_t spg = (nsteps + S - 1) / S;
  const int64_t g0 = ky * spg, g1 = min(nsteps, g0 + spg);
  const int64_t per = g1 > g0 ? (g1 - g0 + NW - 1) / NW : 0;
  const int64_t s0 = g0 + wave * per, s1 = min(g1, s0 + per);
  const bf16x8 zero = {};
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  f32x4 sq = {0.f, 0.f, 0.f, 0.f};  // NORM: X X^T, lane (m, g) holds rows 4 g .. 4 g + 3 of column m
  for (int64_t s = s0; s < s1; s += U) {
    bf16x8 w[U], x[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t k = (s + u) * 32;
      const bool in = s + u < s1 && k + 8 * g < p.K;
      w[u] = in ? *reinterpret_cast<const bf16x8*>(W + k) : zero;
      x[u] = in && xrow ? *reinterpret_cast<const bf16x8*>(X + k) : zero;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[u], x[u], acc, 0, 0, 0);
      if constexpr (NORM) sq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[u], x[u], sq, 0, 0, 0);
    }
  }
  red[wave][lane] = acc;
  if constexpr (NORM) {
    if (g == (r >> 2)) ssq[wave][r] = sq[r & 3];  // the diagonal element (r, r)
  }
  __syncthreads();
  if (S == 1) {
    if (wave == 0 && xrow) {
      f32x4 t = red[0][lane];
#pragma unroll
      for (int w = 1; w < NW; ++w) t += red[w][lane];
      if constexpr (NORM) {
        float q = ssq[0][r];
#pragma unroll
        for (int w = 1; w < NW; ++w) q += ssq[w][r];
        t *= 1.0f / sqrtf(q / (float)p.K + p.norm_eps);
      }
      float v[4] = {t[0], t[1], t[2], t[3]};
      epilogue4<bf16_t, TO>(p, zo, zi, r, n0 + 4 * g, v);
    }
    return;
  }
  // split K (no norm: the host keeps normed products unsplit)
  if (wave == 0) {
    const int64_t tile = (int64_t)blockIdx.z * gridDim.x + blockIdx.x;
    f32x4 t = red[0][lane];
#pragma unroll
    for (int w = 1; w < NW; ++w) t += red[w][lane];
    *reinterpret_cast<f32x4*>(part + ((tile * S + ky) * 64 + lane) * 4) = t;
  }
}

// gemm_skinny_stream_kernel: the few-row product as a persistent weight stream, for K a
// multiple of 2048 (config-5 decode: K = 2048 for QKV, out-projection, GeGLU and the LM head,
// 16384 for the down projection). K is cut into parts of 2048 (gridDim.x = parts x
// workgroups per part, part = blockIdx.x % parts) and a workgroup walks the 16-row blocks of
// Bt n0 = 16 b, b = blockIdx.x / parts, + (gridDim.x / parts), ... Its 4 waves split the
// part's K into 512-wide ranges of 16 steps of 32, one load of Bt per step and wave as in
// gemm_skinny_kernel (lane: row lane % 16, 8 columns at 8 (lane / 16)). The A rows of a
// wave's range are the same for every block, so they are loaded once (and, with norm_rows,
// their X X^T taken once), and the next block's 16 Bt fragments are loaded while the current
// block's 16 MFMAs run: each wave keeps 16 KB of weights in flight across blocks instead of
// letting its loads drain to zero between workgroups. The 4 partial sums of a block meet in
// LDS (two alternating buffers, one barrier per block) and wave 0 runs the epilogue, or, with
// more than one part, writes the block's partial for gemm_skinny_reduce_kernel.
template <typename TO, bool NORM>
__global__ __launch_bounds__(256) void gemm_skinny_stream_kernel(GemmParams p, float* part) {
  constexpr int NW = 4, U = 16, KW = U * 32;  // K per wave per part: 512
  __shared__ f32x4 red[2][NW][64];
  __shared__ float ssq[NW][16];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int r = lane & 15, g = lane >> 4;
  const int S = (int)(p.K / (NW * KW));  // parts
  const int ky = (int)blockIdx.x % S, wpp = (int)gridDim.x / S;
  const int nblk = (int)((p.N + 15) / 16);
  const int64_t k0 = (int64_t)ky * (NW * KW) + wave * KW + 8 * g;
  const bool xrow = r < p.M;
  const bf16_t* X = (const bf16_t*)p.A + (xrow ? r : 0) * p.lda + k0;
  const bf16_t* Bt = (const bf16_t*)p.B + k0;
  const bf16x8 zero = {};
  bf16x8 x[U];
#pragma unroll
  for (int u = 0; u < U; ++u) x[u] = xrow ? *reinterpret_cast<const bf16x8*>(X + u * 32) : zero;
  if constexpr (NORM) {
    f32x4 sq = {0.f, 0.f, 0.f, 0.f};  // X X^T: lane (m, g) holds rows 4 g .. 4 g + 3 of column m
#pragma unroll
    for (int u = 0; u < U; ++u) sq = __builtin_amdgcn_mfma_f32_16x16x32_bf16(x[u], x[u], sq, 0, 0, 0);
    if (g == (r >> 2)) ssq[wave][r] = sq[r & 3];  // the diagonal element (r, r)
  }
  float rscale = 1.f;  // NORM: 1 / rms of row r (wave 0), taken after the first barrier
  bool have_scale = false;
  auto load = [&](bf16x8 (&w)[U], int b) {
    const bf16_t* W = Bt + min((int64_t)b * 16 + r, p.N - 1) * p.ldb;
#pragma unroll
    for (int u = 0; u < U; ++u) w[u] = *reinterpret_cast<const bf16x8*>(W + u * 32);
  };
  int par = 0;
  auto block = [&](const bf16x8 (&w)[U], int b) {
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int u = 0; u < U; ++u) acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(w[u], x[u], acc, 0, 0, 0);
    red[par][wave][lane] = acc;
    __syncthreads();
    if (wave == 0) {
      f32x4 t = red[par][0][lane];
#pragma unroll
      for (int w2 = 1; w2 < NW; ++w2) t += red[par][w2][lane];
      if (S == 1) {
        if constexpr (NORM) {
          if (!have_scale) {  // first block: the row's 1 / rms from the waves' diagonals
            float q = ssq[0][r];
#pragma unroll
            for (int w2 = 1; w2 < NW; ++w2) q += ssq[w2][r];
            rscale = 1.0f / sqrtf(q / (float)p.K + p.norm_eps);
            have_scale = true;
          }
          t *= rscale;
        }
        if (xrow) {
          float v[4] = {t[0], t[1], t[2], t[3]};
          epilogue4<bf16_t, TO>(p, 0, 0, r, (int64_t)b * 16 + 4 * g, v);
        }
      } else {
        *reinterpret_cast<f32x4*>(part + (((int64_t)b * S + ky) * 64 + lane) * 4) = t;
      }
    }
    par ^= 1;
  };
  bf16x8 wa[U], wb[U];
  int b = (int)blockIdx.x / S;
  if (b < nblk) load(wa, b);
  while (b < nblk) {
    const int b1 = b + wpp;
    if (b1 < nblk) load(wb, b1);
    block(wa, b);
    if (b1 >= nblk) break;
    const int b2 = b1 + wpp;
    if (b2 < nblk) load(wa, b2);
    block(wb, b1);
    b = b2;
  }
}

// One wave per 16-row block: sums the `split` partials of the skinny kernel, then the epilogue.
template <typename TO>
__global__ __launch_bounds__(64) void gemm_skinny_reduce_kernel(GemmParams p, const float* part,
                                                                int split) {
  const int lane = threadIdx.x, r = lane & 15, g = lane >> 4;
  if (r >= p.M) return;
  const int64_t z = blockIdx.z;
  const int64_t zo = z / p.batch_inner, zi = z - zo * p.batch_inner;
  const int64_t tile = z * gridDim.x + blockIdx.x;
  f32x4 t = {0.f, 0.f, 0.f, 0.f};
  for (int k = 0; k < split; ++k)
    t += *reinterpret_cast<const f32x4*>(part + ((tile * split + k) * 64 + lane) * 4);
  float v[4] = {t[0], t[1], t[2], t[3]};
  epilogue4<bf16_t, TO>(p, zo, zi, r, (int64_t)blockIdx.x * 16 + 4 * g, v);
}

// 64x64 tiles, 32-wide K steps, 4x4 outputs per thread. The next K step's A and B elements
// are loaded into registers while the current step is computed from LDS, so each step costs
// its FMAs rather than a global-memory round trip (512x128x512: 32 dependent 16-wide steps
// took 54 us).
//
// Split K (part != nullptr): workgroup (tile, blockIdx.y) covers K range [y kc, (y + 1) kc)
// and writes its raw 64x64 sums to part[(z, tile, y)]; gemm_simt_reduce_kernel adds the
// gridDim.y parts in order and runs the epilogue. Used when the tiles alone leave most CUs
// idle and K is long (512x128x512: 16 tiles).
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void gemm_simt_kernel(GemmParams p, float* part, int64_t kc) {
  constexpr int BM = 64, BN = 64, BK = 32;
  constexpr int LA = BM * BK / 256, LB = BN * BK / 256;
  __shared__ float As[BK][BM + 4];
  __shared__ float Bs[BK][BN + 4];
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int64_t z = blockIdx.z;
  const int64_t zo = z / p.batch_inner, zi = z % p.batch_inner;
  const int tile = blockIdx.x;
  const int64_t m0 = (int64_t)(tile / p.tiles_n) * BM;
  const int64_t n0 = (int64_t)(tile % p.tiles_n) * BN;
  const TI* A = (const TI*)p.A + zo * p.sa_o + zi * p.sa_i;
  const TI* B = (const TI*)p.B + zo * p.sb_o + zi * p.sb_i;
  float ra[LA], rb[LB];
  // element e of this thread: A row idx / BK, k idx % BK; B (K x N) k idx / BN, column
  // idx % BN, or (N x K) column idx / BK, k idx % BK; consecutive threads read consecutive
  // addresses in every layout
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int e = 0; e < LA; ++e) {
      const int idx = e * 256 + tid, r = idx / BK, kk = idx % BK;
      const int64_t gm = m0 + r, gk = k0 + kk;
      ra[e] = (gm < p.M && gk < p.K) ? Elem<TI>::load(A + gm * p.lda + gk) : 0.f;
    }
#pragma unroll
    for (int e = 0; e < LB; ++e) {
      const int idx = e * 256 + tid;
      if (p.b_kn) {
        const int kk = idx / BN, c = idx % BN;
        const int64_t gn = n0 + c, gk = k0 + kk;
        rb[e] = (gn < p.N && gk < p.K) ? Elem<TI>::load(B + gk * p.ldb + gn) : 0.f;
      } else {
        const int c = idx / BK, kk = idx % BK;
        const int64_t gn = n0 + c, gk = k0 + kk;
        rb[e] = (gn < p.N && gk < p.K) ? Elem<TI>::load(B + gn * p.ldb + gk) : 0.f;
      }
    }
  };
  auto store = [&]() {
#pragma unroll
    for (int e = 0; e < LA; ++e) {
      const int idx = e * 256 + tid;
      As[idx % BK][idx / BK] = ra[e];
    }
#pragma unroll
    for (int e = 0; e < LB; ++e) {
      const int idx = e * 256 + tid;
      if (p.b_kn) Bs[idx / BN][idx % BN] = rb[e];
      else Bs[idx % BK][idx / BK] = rb[e];
    }
  };
  float acc[4][4] = {};
  const int64_t kb = part ? (int64_t)blockIdx.y * kc : 0;
  const int64_t ke = part ? min(p.K, kb + kc) : p.K;
  load(kb);
  for (int64_t k0 = kb; k0 < ke; k0 += BK) {
    store();
    __syncthreads();
    if (k0 + BK < ke) load(k0 + BK);
#pragma unroll
    for (int kk = 0; kk < BK; ++kk) {
      float a[4], b[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) a[i] = As[kk][ty * 4 + i];
#pragma unroll
      for (int j = 0; j < 4; ++j) b[j] = Bs[kk][tx * 4 + j];
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(a[i], b[j], acc[i][j]);
    }
    __syncthreads();
  }
  if (part) {
    float* dst = part + ((z * gridDim.x + tile) * gridDim.y + blockIdx.y) * (BM * BN);
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<float4*>(dst + (ty * 4 + i) * BN + tx * 4) =
          make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
    return;
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) epilogue4<TI, TO>(p, zo, zi, m0 + ty * 4 + i, n0 + tx * 4, acc[i]);
}

// One workgroup per (z, tile): the `split` partial 64x64 sums in K order, then the epilogue.
template <typename TI, typename TO>
__global__ __launch_bounds__(256) void gemm_simt_reduce_kernel(GemmParams p, const float* part,
                                                               int split) {
  const int tid = threadIdx.x, tx = tid & 15, ty = tid >> 4;
  const int64_t z = blockIdx.z;
  const int64_t zo = z / p.batch_inner, zi = z % p.batch_inner;
  const int tile = blockIdx.x;
  const int64_t m0 = (int64_t)(tile / p.tiles_n) * 64;
  const int64_t n0 = (int64_t)(tile % p.tiles_n) * 64;
  const float* src = part + (z * gridDim.x + tile) * (int64_t)split * 4096;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    float v[4] = {0.f, 0.f, 0.f, 0.f};
    for (int k = 0; k < split; ++k) {
      const float4 t = *reinterpret_cast<const float4*>(src + k * 4096 + (ty * 4 + i) * 64 + tx * 4);
      v[0] += t.x; v[1] += t.y; v[2] += t.z; v[3] += t.w;
    }
    epilogue4<TI, TO>(p, zo, zi, m0 + ty * 4 + i, n0 + tx * 4, v);
  }
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

struct TileShape {
  int bm, bn, threads;
};
static const TileShape kTiles[] = {{0, 0, 0},      {256, 256, 512}, {256, 128, 256},
                                   {128, 128, 256}, {128, 64, 256},  {64, 64, 256},
                                   {256, 256, 256}, {256, 128, 512}, {128, 128, 256},
                                   {256, 128, 512}, {128, 64, 256},  {128, 128, 256},
                                   {256, 128, 512}, {128, 128, 256}, {16, 16, 256},
                                   {256, 256, 512}, {128, 96, 256},  {256, 96, 512},
                                   {256, 96, 512},  {256, 256, 512}, {256, 192, 512}};
static bool is_persistent(int tile) {
  return tile == TL_TILE_PERSIST_256x128_W8 || tile == TL_TILE_PERSIST_128x128 ||
         tile == TL_TILE_PERSIST_256x96_W8 || tile == TL_TILE_PERSIST_256x256_W8;
}
// the non-persistent tile of the same shape
static int persistent_fallback(int tile) {
  switch (tile) {
    case TL_TILE_PERSIST_256x128_W8: return TL_TILE_DMA_256x128_W8;
    case TL_TILE_PERSIST_128x128: return TL_TILE_DMA_128x128;
    case TL_TILE_PERSIST_256x96_W8: return TL_TILE_DMA_256x96_W8;
    default: return TL_TILE_DMA_256x256_W8;
  }
}
// resident workgroups per CU of the persistent variants (LDS: 64 KB for 128x128, 128 KB or
// more for the others)
static int persistent_per_cu(int tile) { return tile == TL_TILE_PERSIST_128x128 ? 2 : 1; }

// Tile choice, from MI355X sweeps of the GPT-2-small (M = 8192) and ViT-S/4 (M = 33280)
// GEMMs and an 8192^3 square: the direct-to-LDS kernels (K % 64 == 0) run best with 256x256
// tiles when there are enough of them, else with 128-row tiles sized to the last round of
// resident workgroups; register-prefetch tiles cover other K; 64x64 covers grids too
// small to fill the GPU.
static int choose_tile(int64_t M, int64_t N, int64_t K, int64_t batch, int cus, bool wide_ok,
                       bool qkv_split) {
  auto tiles = [&](int64_t bm, int64_t bn) { return ((M + bm - 1) / bm) * ((N + bn - 1) / bn) * batch; };
  const int64_t t128 = tiles(128, 128), t64 = tiles(128, 64);
  if (K % 64 == 0) {
    // many 256x256 tiles (LM head, large square): 8 waves of 128x64 read the least LDS and
    // L2 per flop (787 TF on the LM head vs 627; 1335 TF at 8192^3)
    if (tiles(256, 256) >= 4LL * cus) return TL_TILE_DMA_256x256_W8;
    // ... and for a long K loop (K >= 4096, which amortises the tile's start) when they fill
    // at least 90% of their rounds: the config-5 down projection (K = 16384, 256 tiles on 256
    // CUs) 256x128 -> 256x256, prefill 37.92 -> 37.40 ms (same box, two rounds)
    {
      const int64_t t256 = tiles(256, 256), rounds = (t256 + cus - 1) / cus;
      if (K >= 4096 && t256 >= cus && t256 * 10 >= rounds * cus * 9) return TL_TILE_DMA_256x256_W8;
    }
    // 256-row tiles with a 3-stage pipeline (two K steps of loads in flight, one workgroup
    // per CU) when they fill at least one round: inside a forward the weights arrive cold and
    // the activations from the previous kernel, and the deeper pipeline beats two 2-stage
    // 128-row workgroups per CU (GPT-2 prefill 4.06 -> 3.88 ms with 256x128 alone) though
    // it is slower on operands hot in cache. Width 96 or 128, whichever wastes less area in
    // the last round, 128 on a tie (GPT-2: 96 at N = 768 and 2304; at N = 3072 both fill
    // whole rounds and 128's fewer, larger tiles measured 3.79 vs 3.88 ms per forward).
    const int64_t t96w = tiles(256, 96), t128w = tiles(256, 128);
    if (K >= 256 && t96w >= cus) {
      const int64_t w96 = (t96w + cus - 1) / cus * 96, w128 = (t128w + cus - 1) / cus * 128;
      int best = w96 < w128 ? TL_TILE_DMA_256x96_W8 : TL_TILE_DMA_256x128_W8;
      // 192 wide on the same terms, preferred on a tie: 8 waves of 64x96 read a sixth fewer
      // LDS fragment bytes per flop than 64x64 (the inner loop alone 1.86 vs 1.47 PFLOP/s),
      // though only two stages fit the LDS. GPT-2 FFN1 (N = 3072: 2 rounds of 192 against
      // 3 of 128): 54.6 -> 49.1 us behind a warming LayerNorm in a standalone harness. Only
      // for the staged plain / bias / activation / residual epilogues (a 96-column wave slab
      // would straddle QKV parts or GeGLU pairs) and K > 512 (shorter K runs persistent).
      if (wide_ok && K > 512) {
        const int64_t w192 = (tiles(256, 192) + cus - 1) / cus * 192;
        if (w192 <= std::min(w96, w128)) best = TL_TILE_DMA_256x192_W8;
      }
      // The QKV head scatter (K <= 1024) on the two-per-CU 128-row tile of the same width,
      // which takes the same whole rounds (GPT-2 QKV: 768 tiles of 256x96 on 256 CUs, 1536 of
      // 128x96 on 512 slots): one workgroup's scatter epilogue runs under the other's K loop.
      // GPT-2 (256x96 -> 128x96) 3.482 -> 3.450 ms per forward, same box, three alternating
      // rounds (the out-projection on it as well: no further gain); ViT-S/4 (K = 384,
      // 256x128 -> 128x128) 2.284 -> 2.255 ms.
      if (qkv_split && K <= 1024) {
        if (best == TL_TILE_DMA_256x96_W8) best = TL_TILE_DMA_128x96;
        else if (best == TL_TILE_DMA_256x128_W8) best = TL_TILE_DMA_128x128;
      }
      return best;
    }
    // otherwise 128-row tiles, 2 workgroups per CU: the width whose last round of
    // workgroups wastes the least area (N = 768 or 2304: 128x96; 3072: 128x128)
    const int64_t slots = 2LL * cus;
    const int64_t a128 = (t128 + slots - 1) / slots * 128 * 128;
    const int64_t t96 = tiles(128, 96);
    const int64_t a96 = (t96 + slots - 1) / slots * 128 * 96;
    if (t96 >= cus) return a96 < a128 ? TL_TILE_DMA_128x96 : TL_TILE_DMA_128x128;
  }
  // at most 64 rows per product (the ViT patch projection, batched over images, M = 64,
  // K = 48): 128-row tiles would compute half padding (36.6 -> 22.5 us in the model)
  if (M <= 64) return TL_TILE_64x64;
  if (t128 >= 16LL * cus) return TL_TILE_128x128;
  if (t64 >= (int64_t)cus) return TL_TILE_128x64;
  return TL_TILE_64x64;
}

// The streaming form (gemm_skinny_stream_kernel): `parts` K parts of 2048, `wpp` workgroups per
// part (a multiple of nothing: the workgroups of a part stride over its 16-row blocks).
template <typename TO>
static void launch_skinny_stream(int parts, int wpp, int nblk, hipStream_t st, const GemmParams& p,
                                 float* part) {
  const dim3 grid((unsigned)(parts * wpp));
  if (p.norm_rows) gemm_skinny_stream_kernel<TO, true><<<grid, 256, 0, st>>>(p, part);
  else gemm_skinny_stream_kernel<TO, false><<<grid, 256, 0, st>>>(p, part);
  if (parts > 1) gemm_skinny_reduce_kernel<TO><<<dim3((unsigned)nblk, 1, 1), 64, 0, st>>>(p, part, parts);
}

// The per-tile form: 4 waves per workgroup, 16 K steps in flight per wave. On an MI355X at
// the config-5 decode shapes (M = 4) this streamed the wide products fastest of (4, 8),
// (8, 16), (8, 8), (16, 4), (8, 4) and (16, 8) (GeGLU 134 MB in 23.9 us, LM head 1.05 GB in
// 197 us, before the streaming form took those shapes).
template <typename TO>
static void launch_skinny(dim3 grid, hipStream_t st, const GemmParams& p, float* part) {
  if (p.norm_rows) gemm_skinny_kernel<TO, 4, 16, true><<<grid, 256, 0, st>>>(p, part);
  else gemm_skinny_kernel<TO, 4, 16, false><<<grid, 256, 0, st>>>(p, part);
  if (grid.y > 1)
    gemm_skinny_reduce_kernel<TO><<<dim3(grid.x, 1, grid.z), 64, 0, st>>>(p, part, (int)grid.y);
}

template <typename TO>
static void launch_mfma(int tile, dim3 grid, hipStream_t st, const GemmParams& p) {
  switch (tile) {
    case TL_TILE_256x256: gemm_mfma_kernel<TO, 256, 256, 2, 4><<<grid, 512, 0, st>>>(p); break;
    case TL_TILE_256x128: gemm_mfma_kernel<TO, 256, 128, 2, 2><<<grid, 256, 0, st>>>(p); break;
    case TL_TILE_128x128: gemm_mfma_kernel<TO, 128, 128, 2, 2><<<grid, 256, 0, st>>>(p); break;
    case TL_TILE_128x64: gemm_mfma_kernel<TO, 128, 64, 2, 2><<<grid, 256, 0, st>>>(p); break;
    case TL_TILE_256x256_W4: gemm_mfma_kernel<TO, 256, 256, 2, 2><<<grid, 256, 0, st>>>(p); break;
    case TL_TILE_256x128_W8: gemm_mfma_kernel<TO, 256, 128, 4, 2><<<grid, 512, 0, st>>>(p); break;
    case TL_TILE_DMA_128x128: gemm_dma_kernel<TO, 128, 128, 2, 2, 2, 2><<<grid, 256, 0, st>>>(p); break;
    case TL_TILE_DMA_256x128_W8: gemm_dma_kernel<TO, 256, 128, 4, 2, 2, 3><<<grid, 512, 0, st>>>(p); break;
    case TL_TILE_DMA_128x64_S3: gemm_dma_kernel<TO, 128, 64, 2, 2, 2, 3><<<grid, 256, 0, st>>>(p); break;
    case TL_TILE_DMA_128x128_S3: gemm_dma_kernel<TO, 128, 128, 2, 2, 1, 3><<<grid, 256, 0, st>>>(p); break;
    case TL_TILE_DMA_256x256_W8: gemm_dma_kernel<TO, 256, 256, 2, 4, 2, 2><<<grid, 512, 0, st>>>(p); break;
    case TL_TILE_DMA_128x96: gemm_dma_kernel<TO, 128, 96, 2, 2, 2, 2><<<grid, 256, 0, st>>>(p); break;
    case TL_TILE_DMA_256x96_W8: gemm_dma_kernel<TO, 256, 96, 4, 2, 2, 3><<<grid, 512, 0, st>>>(p); break;
    case TL_TILE_DMA_256x192_W8: gemm_dma_kernel<TO, 256, 192, 4, 2, 2, 2><<<grid, 512, 0, st>>>(p); break;
    default: gemm_mfma_kernel<TO, 64, 64, 2, 2><<<grid, 256, 0, st>>>(p); break;
  }
}

// The QKV scatter with element-wise V^T stores (T, L or pos0 not a multiple of 8) on the
// tiles the QKV rule picks.
static void launch_qkv_velem(int tile, dim3 grid, hipStream_t st, const GemmParams& p) {
  if (tile == TL_TILE_DMA_128x96) gemm_dma_kernel<bf16_t, 128, 96, 2, 2, 2, 2, true><<<grid, 256, 0, st>>>(p);
  else gemm_dma_kernel<bf16_t, 128, 128, 2, 2, 2, 2, true><<<grid, 256, 0, st>>>(p);
}

template <int KIND>
static void launch_persistent_kind(int tile, dim3 grid, hipStream_t st, const GemmParams& p) {
  switch (tile) {
    case TL_TILE_PERSIST_256x128_W8: gemm_dma_persistent_kernel<KIND, 256, 128, 4, 2, 2, 3><<<grid, 512, 0, st>>>(p); break;
    case TL_TILE_PERSIST_128x128: gemm_dma_persistent_kernel<KIND, 128, 128, 2, 2, 2, 2><<<grid, 256, 0, st>>>(p); break;
    case TL_TILE_PERSIST_256x96_W8: gemm_dma_persistent_kernel<KIND, 256, 96, 4, 2, 2, 3><<<grid, 512, 0, st>>>(p); break;
    default: gemm_dma_persistent_kernel<KIND, 256, 256, 2, 4, 2, 2><<<grid, 512, 0, st>>>(p); break;
  }
}
static void launch_persistent(int tile, dim3 grid, hipStream_t st, const GemmParams& p) {
  switch (p.epi) {
    case EPI_PLAIN: launch_persistent_kind<EPI_PLAIN>(tile, grid, st, p); break;
    case EPI_BIAS: launch_persistent_kind<EPI_BIAS>(tile, grid, st, p); break;
    case EPI_BIAS_GELU: launch_persistent_kind<EPI_BIAS_GELU>(tile, grid, st, p); break;
    case EPI_BIAS_SILU: launch_persistent_kind<EPI_BIAS_SILU>(tile, grid, st, p); break;
    case EPI_BIAS_RES: launch_persistent_kind<EPI_BIAS_RES>(tile, grid, st, p); break;
    default: launch_persistent_kind<EPI_RES>(tile, grid, st, p); break;
  }
}

}  // namespace tl

using namespace tl;

extern "C" int tl_gemm(tl_ctx* ctx, const tl_gemm_desc* d) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(d, "null descriptor");
  TL_REQUIRE(d->M > 0 && d->N > 0 && d->K > 0, "GEMM sizes must be positive (M=%lld N=%lld K=%lld)",
             (long long)d->M, (long long)d->N, (long long)d->K);
  TL_REQUIRE(d->M < (1LL << 31) && d->N < (1LL << 31), "M and N must be below 2^31");
  TL_REQUIRE(d->A && d->B, "null operand");
  TL_REQUIRE(dtype_is_float(d->dtype_in) && dtype_is_float(d->dtype_out), "GEMM dtypes must be fp32 or bf16");
  TL_REQUIRE(d->b_layout == TL_B_NK || d->b_layout == TL_B_KN, "bad b_layout %d", d->b_layout);
  TL_REQUIRE(d->act == TL_ACT_NONE || d->act == TL_ACT_GELU || d->act == TL_ACT_SILU, "bad activation");
  TL_REQUIRE(d->divisor != 0.f, "divisor must be non-zero");
  TL_REQUIRE(d->tile >= 0 && d->tile <= TL_TILE_DMA_256x192_W8, "bad tile hint %d", d->tile);
  const int64_t batch = d->batch <= 0 ? 1 : d->batch;
  const int64_t binner = d->batch_inner <= 0 ? 1 : d->batch_inner;
  TL_REQUIRE(batch <= 65535, "batch %lld exceeds 65535", (long long)batch);
  TL_REQUIRE(d->lda >= d->K, "lda < K");
  TL_REQUIRE(d->b_layout == TL_B_NK ? d->ldb >= d->K : d->ldb >= d->N, "ldb too small");
  const bool qkv = d->epilogue == TL_EPI_QKV_SPLIT;
  const bool geglu = d->epilogue == TL_EPI_GEGLU;
  TL_REQUIRE(d->epilogue == TL_EPI_STORE || qkv || geglu, "bad epilogue %d", d->epilogue);
  if (geglu) {
    TL_REQUIRE(d->N % 2 == 0 && !d->residual, "gated epilogue needs even N and no residual");
    TL_REQUIRE(d->act == TL_ACT_GELU || d->act == TL_ACT_SILU, "gated epilogue needs GeLU or SiLU");
  }
  if (qkv) {
    TL_REQUIRE(d->q && d->k && d->vt, "QKV split needs q, k and vt");
    TL_REQUIRE(batch == 1 && !d->residual, "QKV split is unbatched and has no residual");
    TL_REQUIRE(d->seq_len > 0 && d->M % d->seq_len == 0, "M must be a multiple of seq_len");
    TL_REQUIRE(d->head_dim > 0 && d->head_dim % 4 == 0 && d->n_heads_q > 0 &&
                   d->n_heads_kv > 0 && d->n_heads_q % d->n_heads_kv == 0,
               "bad head configuration (head_dim must be a multiple of 4)");
    TL_REQUIRE(d->N == (d->n_heads_q + 2 * d->n_heads_kv) * d->head_dim, "N != (Hq + 2 Hkv) * Dh");
    TL_REQUIRE(d->seq_len < (1LL << 31) && d->N * d->seq_len < (1LL << 40), "QKV split too large");
    const int64_t L = d->kv_len > 0 ? d->kv_len : d->seq_len;
    TL_REQUIRE(d->kv_pos0 >= 0 && d->kv_pos0 + d->seq_len <= L && L < (1LL << 31),
               "cache write [kv_pos0, kv_pos0 + seq_len) exceeds kv_len");
    TL_REQUIRE(!d->kv_pos0_dev || ((uintptr_t)d->kv_pos0_dev % 8 == 0 && d->kv_pos0 == 0),
               "kv_pos0_dev must be an aligned int64 and kv_pos0 0");
  } else {
    TL_REQUIRE(d->C, "null output");
    TL_REQUIRE(d->ldc >= (geglu ? d->N / 2 : d->N), "ldc too small");
  }
  if (d->residual) TL_REQUIRE(d->ldr >= d->N, "ldr < N");

  GemmParams p;
  p.A = d->A; p.B = d->B; p.C = d->C;
  p.M = d->M; p.N = d->N; p.K = d->K; p.lda = d->lda; p.ldb = d->ldb; p.ldc = d->ldc;
  p.batch_inner = binner;
  p.sa_o = d->sa_o; p.sa_i = d->sa_i; p.sb_o = d->sb_o; p.sb_i = d->sb_i;
  p.sc_o = d->sc_o; p.sc_i = d->sc_i;
  p.bias = d->bias; p.res = d->residual; p.ldr = d->ldr; p.sr_o = d->sr_o; p.sr_i = d->sr_i;
  p.divisor = d->divisor; p.act = d->act; p.b_kn = d->b_layout == TL_B_KN;
  p.qkv = qkv; p.q = d->q; p.k = d->k; p.vt = d->vt;
  p.T = (int)d->seq_len; p.Hq = (int)d->n_heads_q; p.Hkv = (int)d->n_heads_kv; p.Dh = (int)d->head_dim;
  p.L = (int)(d->kv_len > 0 ? d->kv_len : d->seq_len);
  p.pos0 = (int)d->kv_pos0;
  p.pos0_dev = qkv ? (const int64_t*)d->kv_pos0_dev : nullptr;
  p.geglu = geglu;
  const size_t eo = dtype_size(d->dtype_out);
  p.vec_store = !qkv && d->ldc % 4 == 0 && ((uintptr_t)d->C % (4 * eo)) == 0 &&
                d->sc_o % 4 == 0 && d->sc_i % 4 == 0;
  if (geglu) p.vec_store = d->ldc % 2 == 0 && ((uintptr_t)d->C % (2 * eo)) == 0 &&
                           d->sc_o % 2 == 0 && d->sc_i % 2 == 0;
  p.vec_res = d->residual && d->ldr % 4 == 0 && ((uintptr_t)d->residual % (4 * eo)) == 0 &&
              d->sr_o % 4 == 0 && d->sr_i % 4 == 0;
  // LDS-staged epilogue: bf16 rows that take 16-byte stores, residual rows that take 8-byte
  // loads (N % 4 == 0), no divisor; the other combinations use the generic epilogue
  p.epi = EPI_GENERIC;
  const bool st16 = !qkv && !geglu && eo == 2 && d->ldc % 8 == 0 && ((uintptr_t)d->C % 16) == 0 &&
                    d->sc_o % 8 == 0 && d->sc_i % 8 == 0 && d->divisor == 1.0f;
  const bool res_ok = !d->residual || (p.vec_res && d->N % 4 == 0);
  if (st16 && res_ok) {
    const bool b = d->bias != nullptr, r = d->residual != nullptr;
    if (!b && !r && d->act == TL_ACT_NONE) p.epi = EPI_PLAIN;
    else if (b && !r && d->act == TL_ACT_NONE) p.epi = EPI_BIAS;
    else if (b && !r && d->act == TL_ACT_GELU) p.epi = EPI_BIAS_GELU;
    else if (b && !r && d->act == TL_ACT_SILU) p.epi = EPI_BIAS_SILU;
    else if (b && r && d->act == TL_ACT_NONE) p.epi = EPI_BIAS_RES;
    else if (!b && r && d->act == TL_ACT_NONE) p.epi = EPI_RES;
  }
  // The staged QKV scatter: 16-byte V^T units need T, L and pos0 multiples of 8; otherwise
  // the two-per-CU 128-row tiles the QKV rule picks take the element-wise V^T form
  // (qkv_velem, decided with the tile) and other tiles the generic epilogue.
  const bool qkv_staged = qkv && !d->kv_pos0_dev && eo == 2 && d->divisor == 1.0f &&
                          d->act == TL_ACT_NONE && !d->residual && d->head_dim % 8 == 0 &&
                          ((uintptr_t)d->q % 16) == 0 && ((uintptr_t)d->k % 16) == 0 &&
                          ((uintptr_t)d->vt % 16) == 0;
  const bool qkv_aligned = d->seq_len % 8 == 0 && p.L % 8 == 0 && p.pos0 % 8 == 0;
  if (qkv_staged && qkv_aligned) p.epi = d->bias ? EPI_QKV_BIAS : EPI_QKV;
  if (geglu && eo == 2 && !d->bias && d->divisor == 1.0f && (d->N / 2) % 8 == 0 && d->ldc % 8 == 0 &&
      ((uintptr_t)d->C % 16) == 0 && d->sc_o % 8 == 0 && d->sc_i % 8 == 0)
    p.epi = d->act == TL_ACT_GELU ? EPI_GEGLU_GELU : EPI_GEGLU_SILU;
  // Tile-rows per group, measured in-model: 6 beats 3/5/7/8/10 on GPT-2 (3.422 vs 3.456 ms at
  // 8; every GPT-2 product is fastest at 6) and ties on ViT-S/4; 16 and 32 lose 3-17%. The
  // config-5 vocabulary product (K = 2048, 1000 tile-columns of 256) runs best at 8 (7291 ->
  // 6766 us in a kernel trace; 4 is close, 2 and 3 slower; config-5 prefill 37.45 -> 37.16 ms,
  // same box, three alternating rounds), while the config-5 GeGLU product (K = 2048, 128
  // tile-columns) lost 0.8 ms per prefill at 8 in-model.
  p.group_m = d->K >= 2048 && d->K < 4096 && d->N >= 512 * 256 ? 8 : 6;
  p.div_T = make_fastdiv(qkv ? (uint32_t)d->seq_len : 1u);
  p.div_Dh = make_fastdiv(qkv ? (uint32_t)d->head_dim : 1u);
  p.norm_rows = d->norm_rows != 0;
  p.norm_eps = d->norm_eps;

  // The MFMA kernel streams 16-byte rows of A and Bt: K-contiguous, 8-element aligned.
  const bool mfma = d->dtype_in == TL_BF16 && d->b_layout == TL_B_NK && d->K % 8 == 0 &&
                    d->lda % 8 == 0 && d->ldb % 8 == 0 && d->sa_o % 8 == 0 &&
                    d->sa_i % 8 == 0 && d->sb_o % 8 == 0 && d->sb_i % 8 == 0 && al16(d->A) &&
                    al16(d->B);
  const double es_in = (double)dtype_size(d->dtype_in);
  const double flops = 2.0 * d->M * d->N * d->K * batch;
  const double bytes = batch * (es_in * ((double)d->M * d->K + (double)d->N * d->K) +
                                (double)eo * d->M * d->N * (d->residual ? 2 : 1));
  // fp32 operands on the matrix cores under the same layout rules (4-element alignment) when
  // there are at least 128 output tiles of 128x128; fewer stay on the split-K VALU kernel.
  const bool mfma32_layout = d->dtype_in == TL_F32 && d->b_layout == TL_B_NK && d->K % 4 == 0 &&
                             d->lda % 4 == 0 && d->ldb % 4 == 0 && d->sa_o % 4 == 0 &&
                             d->sa_i % 4 == 0 && d->sb_o % 4 == 0 && d->sb_i % 4 == 0 &&
                             al16(d->A) && al16(d->B) && d->lda * 128 < (1LL << 31) &&
                             d->ldb * 128 < (1LL << 31);
  const bool mfma32 = mfma32_layout && ((d->M + 127) / 128) * ((d->N + 127) / 128) * batch >= 128;
  // small fp32 products with a short K loop (the char-level GPT: M = 512, K = 128 .. 512)
  // on 64x64 fp32 MFMA tiles rather than the vector ALUs; long K with few tiles stays on the
  // split-K vector kernel
  const bool mfma32_small = mfma32_layout && !mfma32 && d->K <= 1024 &&
                            ((d->M + 63) / 64) * ((d->N + 63) / 64) * batch >= 8;
  const int family = (mfma || mfma32 || mfma32_small) ? d->family : TL_KF_GEMM_SIMT;
  TL_REQUIRE(family >= 0 && family < TL_KF_COUNT, "bad kernel family");
  const bool f32out = d->dtype_out == TL_F32;
  const bool skinny = mfma && (d->tile == TL_TILE_SKINNY || (d->tile == TL_TILE_AUTO && d->M <= 16));
  if (d->norm_rows) {
    if (!skinny || batch != 1)
      return fail(TL_ERR_UNSUPPORTED, "RMS row scaling is implemented for unbatched bf16 "
                  "products with M <= 16 and B as [N, K]");
    TL_REQUIRE(d->norm_eps >= 0.f, "norm_eps must be >= 0");
  }
  if (skinny) {
    TL_REQUIRE(d->M <= 16, "the skinny GEMM takes M <= 16");
    const int64_t tiles = (d->N + 15) / 16 * batch;
    const int64_t nsteps = (d->K + 31) / 32;
    const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    // K a multiple of 2048, one product: the persistent weight stream, K in parts of 2048 (a
    // second launch sums the parts when there is more than one; the row-scaled form takes
    // one part). One workgroup per CU for one part (config-5 decode 1.485 -> 1.473 ms per step
    // against two: GeGLU's 2048 blocks run 8 per workgroup instead of 4, with less start-up
    // and tail per byte), two per CU (two waves per SIMD: ~230 VGPRs) over several parts.
    const int64_t parts = d->K / 2048;
    if (batch == 1 && d->K % 2048 == 0 && parts <= 64 && tiles < (1LL << 30) &&
        (!d->norm_rows || parts == 1)) {
      const int64_t wpp = std::max<int64_t>(1, std::min<int64_t>(tiles, (parts == 1 ? 1 : 2) * cus / parts));
      float* part = nullptr;
      if (parts > 1) {
        void* ws;
        rc = workspace(ctx, (size_t)tiles * parts * 64 * 4 * sizeof(float), &ws);
        if (rc) return rc;
        part = (float*)ws;
      }
      LaunchScope ls(ctx, family, flops, bytes);
      if (f32out) launch_skinny_stream<float>((int)parts, (int)wpp, (int)tiles, ctx->stream, p, part);
      else launch_skinny_stream<bf16_t>((int)parts, (int)wpp, (int)tiles, ctx->stream, p, part);
      return ls.finish("gemm_skinny_stream");
    }
    // Long K only (the split costs a second launch): split until there are 2 workgroups
    // per CU while every part keeps >= 4096 of K (down projection K = 16384: 4 parts,
    // 23.6 -> 18.0 us; K = 2048 shapes lose more to the extra launch than they gain).
    int64_t split = 1;
    while (!d->norm_rows && split < 16 &&
           tiles * split < 2 * cus && nsteps / (split * 2) >= 128)
      split *= 2;
    dim3 grid((unsigned)((d->N + 15) / 16), (unsigned)split, (unsigned)batch);
    float* part = nullptr;
    if (split > 1) {
      void* ws;
      rc = workspace(ctx, (size_t)tiles * split * 64 * 4 * sizeof(float), &ws);
      if (rc) return rc;
      part = (float*)ws;
    }
    LaunchScope ls(ctx, family, flops, bytes);
    if (f32out) launch_skinny<float>(grid, ctx->stream, p, part);
    else launch_skinny<bf16_t>(grid, ctx->stream, p, part);
    return ls.finish("gemm_skinny");
  }
  if (mfma) {
    const int cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    const bool wide_ok = !f32out && p.epi >= EPI_PLAIN && p.epi <= EPI_RES;
    int tile = d->tile ? d->tile : choose_tile(d->M, d->N, d->K, batch, cus, wide_ok, qkv);
    const bool fixed = d->tile != 0;  // a caller's tile is kept as is
    if (tile >= TL_TILE_DMA_128x128 && d->K % 64 != 0) tile = TL_TILE_128x128;  // DMA needs whole K steps
    // the persistent kernels store through a buffer resource: whole 16-byte pieces, byte
    // offsets below 2^31
    const bool persist_ok = batch == 1 && !f32out && p.epi >= EPI_PLAIN && p.epi <= EPI_RES &&
                            d->N % 8 == 0 && ((d->M - 1) * d->ldc + d->N) * 2 < (int64_t)0x7fffffff;
    if (is_persistent(tile) && !persist_ok) tile = persistent_fallback(tile);
    // Automatic choice: with a K loop of at most 8 steps and two or more tiles per CU, the
    // next tile's first loads pay off when issued under the current tile's epilogue
    // (ViT-S/4 FFN1 +12%, out-proj +5%); at K = 768 the two variants tie and with one tile
    // per CU the persistent bookkeeping costs 4-10%.
    // With at least 8 tiles of 128x128 per CU the two-per-CU persistent 128x128 tile walks
    // 6+ tiles per workgroup and beats the 256-row persistent ones inside the model
    // (ViT-S/4 FFN1, 33280 x 1536, K = 384: 2.77 -> 2.69 ms per forward; out-proj, 1.5 tiles
    // per workgroup, is slower on it).
    const int64_t t128 = ((d->M + 127) / 128) * ((d->N + 127) / 128);
    if (!fixed && persist_ok && d->K <= 512 && d->K % 64 == 0 && t128 >= 8LL * cus) {
      tile = TL_TILE_PERSIST_128x128;
    } else if (!fixed && persist_ok && d->K <= 512 &&
               (tile == TL_TILE_DMA_256x96_W8 || tile == TL_TILE_DMA_256x128_W8)) {
      const TileShape& t = kTiles[tile];
      const int64_t nt = ((d->M + t.bm - 1) / t.bm) * ((d->N + t.bn - 1) / t.bn);
      if (nt >= 2LL * cus)
        tile = tile == TL_TILE_DMA_256x96_W8 ? TL_TILE_PERSIST_256x96_W8 : TL_TILE_PERSIST_256x128_W8;
    } else if (!fixed && persist_ok && (p.epi == EPI_BIAS_GELU || p.epi == EPI_BIAS_SILU) &&
               d->K % 64 == 0 && d->K <= 1024 && t128 >= 4LL * cus) {
      // An activation epilogue (one exp2 and one reciprocal per element) is vector-ALU bound;
      // on the two-per-CU persistent 128x128 tile one workgroup's epilogue runs under the
      // other's K loop. GPT-2 FFN1 (K = 768, 1536 tiles): 3.337 -> 3.299 ms per forward
      // against 256x192 (same box, three alternating rounds; the persistent 256x128 / 256x96
      // / 256x256 tiles 3.319 / 3.377 / 3.415 ms).
      tile = TL_TILE_PERSIST_128x128;
    }
    // ViT-S/4 QKV (T = 65, 128x128) against the generic epilogue: 2.312 -> 2.221 ms per ViT
    // forward (same box, six alternating pairs); GPT-2 within run-to-run spread
    const bool qkv_velem = qkv_staged && !qkv_aligned &&
                           (tile == TL_TILE_DMA_128x96 || tile == TL_TILE_DMA_128x128);
    if (qkv_velem) p.epi = d->bias ? EPI_QKV_BIAS : EPI_QKV;
    const bool persistent = is_persistent(tile);
    const TileShape& s = kTiles[tile];
    p.tiles_m = (int)((d->M + s.bm - 1) / s.bm);
    p.tiles_n = (int)((d->N + s.bn - 1) / s.bn);
    TL_REQUIRE((int64_t)p.tiles_m * p.tiles_n < 0x7fffffff, "too many tiles");
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
    if (persistent) {
      const int64_t slots = (int64_t)(ctx->num_cus > 0 ? ctx->num_cus : 256) * persistent_per_cu(tile);
      const int64_t ntiles = (int64_t)p.tiles_m * p.tiles_n;
      grid.x = (unsigned)(std::min(slots, (ntiles + 7) / 8 * 8) / 8 * 8);
      if (grid.x == 0) grid.x = 8;
    }
    LaunchScope ls(ctx, family, flops, bytes);
    if (persistent) launch_persistent(tile, grid, ctx->stream, p);
    else if (qkv_velem) launch_qkv_velem(tile, grid, ctx->stream, p);
    else if (f32out) launch_mfma<float>(tile, grid, ctx->stream, p);
    else launch_mfma<bf16_t>(tile, grid, ctx->stream, p);
    return ls.finish("gemm_mfma");
  }
  if (mfma32) {
    // 16-wide K steps: 32 KB of LDS (128x128), so three workgroups share a CU (registers
    // allow three waves per SIMD), and tiles 128 or 64 wide (a load pass covers 64 rows),
    // whichever takes less rounds x width over 3 x CUs slots, 128 unless 64 saves >= 10%
    const int64_t slots = 3 * (int64_t)(ctx->num_cus > 0 ? ctx->num_cus : 256);
    auto round_width = [&](int64_t bn) {
      const int64_t tiles = ((d->M + 127) / 128) * ((d->N + bn - 1) / bn) * batch;
      return (tiles + slots - 1) / slots * bn;
    };
    const int bn = round_width(64) * 10 <= round_width(128) * 9 ? 64 : 128;
    p.tiles_m = (int)((d->M + 127) / 128);
    p.tiles_n = (int)((d->N + bn - 1) / bn);
    TL_REQUIRE((int64_t)p.tiles_m * p.tiles_n < 0x7fffffff, "too many tiles");
    const dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
    LaunchScope ls(ctx, family, flops, bytes);
    if (bn == 64) {
      if (f32out) gemm_mfma_f32_kernel<float, 128, 64, 2, 2, 16><<<grid, 256, 0, ctx->stream>>>(p);
      else gemm_mfma_f32_kernel<bf16_t, 128, 64, 2, 2, 16><<<grid, 256, 0, ctx->stream>>>(p);
    } else {
      if (f32out) gemm_mfma_f32_kernel<float, 128, 128, 2, 2, 16><<<grid, 256, 0, ctx->stream>>>(p);
      else gemm_mfma_f32_kernel<bf16_t, 128, 128, 2, 2, 16><<<grid, 256, 0, ctx->stream>>>(p);
    }
    return ls.finish("gemm_mfma_f32");
  }
  if (mfma32_small) {
    p.tiles_m = (int)((d->M + 63) / 64);
    p.tiles_n = (int)((d->N + 63) / 64);
    const dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
    LaunchScope ls(ctx, family, flops, bytes);
    if (f32out) gemm_mfma_f32_kernel<float, 64, 64, 2, 2><<<grid, 256, 0, ctx->stream>>>(p);
    else gemm_mfma_f32_kernel<bf16_t, 64, 64, 2, 2><<<grid, 256, 0, ctx->stream>>>(p);
    return ls.finish("gemm_mfma_f32_small");
  }
  p.tiles_m = (int)((d->M + 63) / 64);
  p.tiles_n = (int)((d->N + 63) / 64);
  TL_REQUIRE((int64_t)p.tiles_m * p.tiles_n < 0x7fffffff, "too many tiles");
  dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
  // Split K (K >= 256) over workgroups while the parts still fit in one round on the CUs and
  // each keeps at least two 32-wide K steps (512x128x512: 16 tiles x 8 parts).
  const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
  const int64_t tiles = (int64_t)grid.x * batch;
  int64_t split = 1;
  while (d->K >= 256 && split < 16 && tiles * split * 2 <= cus && d->K / (split * 2) >= 64)
    split *= 2;
  float* part = nullptr;
  int64_t kc = d->K;
  if (split > 1) {
    kc = ((d->K + split - 1) / split + 31) / 32 * 32;
    split = (d->K + kc - 1) / kc;
    void* ws;
    rc = workspace(ctx, (size_t)tiles * split * 4096 * sizeof(float), &ws);
    if (rc) return rc;
    part = (float*)ws;
    grid.y = (unsigned)split;
  }
  LaunchScope ls(ctx, family, flops, bytes);
  auto go = [&](auto ti, auto to) {
    using TI = decltype(ti);
    using TO = decltype(to);
    gemm_simt_kernel<TI, TO><<<grid, 256, 0, ctx->stream>>>(p, part, kc);
    if (part)
      gemm_simt_reduce_kernel<TI, TO><<<dim3(grid.x, 1, grid.z), 256, 0, ctx->stream>>>(
          p, part, (int)split);
  };
  if (d->dtype_in == TL_F32) {
    if (f32out) go(float(), float());
    else go(float(), bf16_t());
  } else {
    if (f32out) go(bf16_t(), float());
    else go(bf16_t(), bf16_t());
  }
  return ls.finish("gemm_simt");
}

namespace tl {

// vit_project_kernel: the ViT front end (VitProjector.forward) in one launch, one workgroup
// of 4 waves per image. The image's L <= 64 patch rows are gathered into LDS (features in
// (row in patch, column in patch, channel) order, zero past K <= 64; 16-byte chunks
// XOR-swizzled by row). Each wave takes 96-column groups of the projection (given as
// [E, K], K-contiguous) and, per 16-row tile, issues the same two 16x16x32 MFMA steps with
// the same operand order and zero-filled K tail as the tiled GEMM, adds the row's position
// (after the GEMM epilogue's zero bias) in fp32 and rounds once, so each value equals the
// three-launch path (patch gather, batched GEMM with the positions as residual, class-row
// gather) bit for bit. The 16 x 96 results go through the wave's LDS region and out as
// 16-byte row pieces. Rows 0 .. R-1 are the class/register tokens plus their positions.
__global__ __launch_bounds__(256) void vit_project_kernel(const bf16_t* __restrict__ x,
                                                          const bf16_t* __restrict__ w,
                                                          const bf16_t* __restrict__ cls_reg,
                                                          const bf16_t* __restrict__ pos,
                                                          bf16_t* __restrict__ out, int C, int H,
                                                          int W, int p0, int p1, int E, int R) {
  constexpr int KP = 64, TN = 6, GW = 16 * TN;  // padded K, column tiles per wave group
  __shared__ __attribute__((aligned(16))) bf16_t P[64 * KP];
  __shared__ __attribute__((aligned(16))) bf16_t S[4][16 * GW];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, fc = lane >> 4;
  const int64_t b = blockIdx.x;
  const int pw = W / p1, L = (H / p0) * pw, K = p0 * p1 * C, T = R + L;
  const bf16_t* xi = x + b * C * H * W;
  bf16_t* ob = out + b * T * E;
  for (int idx = tid; idx < 64 * KP; idx += 256) {
    const int l = idx >> 6, t = idx & 63;
    bf16_t v = 0;
    if (l < L && t < K) {
      const int ch = t % C, t2 = t / C, c2 = t2 % p1, a = t2 / p1;
      const int i = l / pw, j = l - i * pw;
      v = xi[((int64_t)ch * H + i * p0 + a) * W + j * p1 + c2];
    }
    P[l * KP + ((((t >> 3) ^ (l & 7))) << 3) + (t & 7)] = v;
  }
  // class/register rows: token + position
  for (int idx = tid; idx < R * E / 4; idx += 256) {
    const int r = idx / (E / 4), c = (idx - r * (E / 4)) * 4;
    const uint2 u = gload8(cls_reg + (int64_t)r * E + c), q = gload8(pos + (int64_t)r * E + c);
    float v[4] = {__uint_as_float(u.x << 16) + __uint_as_float(q.x << 16),
                  __uint_as_float(u.x & 0xffff0000u) + __uint_as_float(q.x & 0xffff0000u),
                  __uint_as_float(u.y << 16) + __uint_as_float(q.y << 16),
                  __uint_as_float(u.y & 0xffff0000u) + __uint_as_float(q.y & 0xffff0000u)};
    gstore8(ob + (int64_t)r * E + c, make_uint2((uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16),
                                                (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16)));
  }
  __syncthreads();
  const bf16x8 zero = {};
  bf16_t* reg = S[wave];
  for (int n0 = wave * GW; n0 < E; n0 += 4 * GW) {
    bf16x8 bfr[2][TN];
#pragma unroll
    for (int s = 0; s < 2; ++s)
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int k = 32 * s + 8 * fc;
        bfr[s][j] = k < K ? gload(reinterpret_cast<const bf16x8*>(w + (int64_t)(n0 + 16 * j + fr) * K + k))
                          : zero;
      }
    for (int i = 0; i < 4 && 16 * i < L; ++i) {
      const int r = 16 * i + fr;
      bf16x8 af[2];
#pragma unroll
      for (int s = 0; s < 2; ++s)
        af[s] = *reinterpret_cast<const bf16x8*>(&P[r * KP + (((s * 4 + fc) ^ (fr & 7)) << 3)]);
      f32x4 acc[TN];
#pragma unroll
      for (int j = 0; j < TN; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2; ++s)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[s][j], af[s], acc[j], 0, 0, 0);
      // row r's position (rows past L read row L - 1 and are not stored)
      const bf16_t* prow = pos + (int64_t)(R + min(r, L - 1)) * E + n0;
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const uint2 q = gload8(prow + 16 * j + 4 * fc);
        const float v0 = (acc[j][0] + 0.f) + __uint_as_float(q.x << 16);
        const float v1 = (acc[j][1] + 0.f) + __uint_as_float(q.x & 0xffff0000u);
        const float v2 = (acc[j][2] + 0.f) + __uint_as_float(q.y << 16);
        const float v3 = (acc[j][3] + 0.f) + __uint_as_float(q.y & 0xffff0000u);
        *reinterpret_cast<uint2*>(&reg[fr * GW + 16 * j + 4 * fc]) =
            make_uint2((uint32_t)f2bf(v0) | ((uint32_t)f2bf(v1) << 16),
                       (uint32_t)f2bf(v2) | ((uint32_t)f2bf(v3) << 16));
      }
      // 16 rows x 12 pieces of 16 bytes; a wave's LDS operations complete in order
#pragma unroll
      for (int p = 0; p < 3; ++p) {
        const int q = p * 64 + lane, rr = q / 12, u = q - rr * 12;
        const uint4 v = *reinterpret_cast<const uint4*>(&reg[rr * GW + 8 * u]);
        if (16 * i + rr < L) gstore16(ob + (int64_t)(R + 16 * i + rr) * E + n0 + 8 * u, v);
      }
    }
  }
}

}  // namespace tl

extern "C" int tl_vit_project(tl_ctx* ctx, const void* x, const void* w, const void* cls_reg,
                              const void* pos, void* out, int64_t batch, int64_t channels,
                              int64_t height, int64_t width, int64_t patch_h, int64_t patch_w,
                              int64_t dim, int64_t n_cls_reg, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(x && w && cls_reg && pos && out, "null pointer");
  TL_REQUIRE(batch > 0 && batch < (1LL << 31) && channels > 0 && patch_h > 0 && patch_w > 0 &&
                 height > 0 && width > 0 && height % patch_h == 0 && width % patch_w == 0,
             "bad image or patch shape");
  TL_REQUIRE(n_cls_reg >= 0 && dim > 0, "bad token shape");
  const int64_t K = patch_h * patch_w * channels, L = (height / patch_h) * (width / patch_w);
  if (dtype != TL_BF16 || K > 64 || K % 8 != 0 || L > 64 || dim % 96 != 0 || dim > 4096 ||
      n_cls_reg > 64 || channels * height * width > (1LL << 24) || !al16(w) || !al16(out) ||
      dim % 8 != 0 || (uintptr_t)cls_reg % 8 != 0 || (uintptr_t)pos % 8 != 0)
    return fail(TL_ERR_UNSUPPORTED, "tl_vit_project takes bf16, K = ph pw C <= 64 (a multiple of "
                "8), at most 64 patches, dim a multiple of 96 and aligned rows");
  const double bytes = 2.0 * (double)batch * (channels * height * width + (L + n_cls_reg) * dim);
  LaunchScope ls(ctx, TL_KF_GEMM_BATCHED, 2.0 * batch * L * dim * K, bytes);
  vit_project_kernel<<<dim3((unsigned)batch), 256, 0, ctx->stream>>>(
      (const bf16_t*)x, (const bf16_t*)w, (const bf16_t*)cls_reg, (const bf16_t*)pos, (bf16_t*)out,
      (int)channels, (int)height, (int)width, (int)patch_h, (int)patch_w, (int)dim, (int)n_cls_reg);
  return ls.finish("vit_project");
}
