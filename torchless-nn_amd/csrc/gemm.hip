// GEMMs of the forward path: C = epilogue(A * op(B)), batched and strided.
//
// gemm_mfma_kernel: bf16 operands, fp32 accumulation on the gfx950 matrix cores
//   (v_mfma_f32_16x16x32_bf16). A is [M, K] and B is given K-contiguous as Bt [N, K], so
//   both tiles stream from HBM as 16-byte rows. BM x BN x 64 tiles are double-buffered in
//   LDS (one barrier per K step); 16-byte chunks are XOR-swizzled by row so the fragment
//   reads of 16 consecutive rows hit distinct banks. The MFMA is issued with Bt as its
//   first operand, so the 16x16 result tile lands transposed: each lane holds 4 consecutive
//   output columns of one row, which the epilogue stores as one 8- or 16-byte write.
// gemm_simt_kernel: any dtype, layout or alignment, fp32 FMA on the vector ALUs. It
//   serves the fp32 model and shapes the MFMA kernel's 16-byte loads cannot take.
#include <algorithm>

#include "tl_internal.hpp"

namespace tl {

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
  int qkv;
  void* q;
  void* k;
  void* vt;
  int64_t T, Hq, Hkv, Dh;
  int tiles_m, tiles_n;
};

// Applies the epilogue to 4 consecutive columns n0..n0+3 of row m and stores them.
template <typename TI, typename TO>
__device__ __forceinline__ void epilogue4(const GemmParams& p, int64_t zo, int64_t zi, int64_t m,
                                          int64_t n0, float v[4]) {
  if (m >= p.M || n0 >= p.N) return;
  const int cnt = p.N - n0 >= 4 ? 4 : (int)(p.N - n0);
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    if (p.divisor != 1.0f) v[e] = v[e] / p.divisor;
    if (p.bias && e < cnt) v[e] = v[e] + Elem<TI>::load((const TI*)p.bias + n0 + e);
    v[e] = apply_act(v[e], p.act);
  }
  if (p.res) {
    const TO* r = (const TO*)p.res + zo * p.sr_o + zi * p.sr_i + m * p.ldr + n0;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      if (e < cnt) v[e] = v[e] + Elem<TO>::load(r + e);
  }
  if (p.qkv) {
    const int64_t b = m / p.T, t = m % p.T;
    const int64_t qw = p.Hq * p.Dh, kw = p.Hkv * p.Dh;
    for (int e = 0; e < cnt; ++e) {
      const int64_t n = n0 + e;
      if (n < qw) {
        const int64_t h = n / p.Dh, d = n % p.Dh;
        Elem<TO>::store((TO*)p.q + ((b * p.Hq + h) * p.T + t) * p.Dh + d, v[e]);
      } else if (n < qw + kw) {
        const int64_t h = (n - qw) / p.Dh, d = (n - qw) % p.Dh;
        Elem<TO>::store((TO*)p.k + ((b * p.Hkv + h) * p.T + t) * p.Dh + d, v[e]);
      } else {
        const int64_t h = (n - qw - kw) / p.Dh, d = (n - qw - kw) % p.Dh;
        Elem<TO>::store((TO*)p.vt + ((b * p.Hkv + h) * p.Dh + d) * p.T + t, v[e]);
      }
    }
    return;
  }
  TO* c = (TO*)p.C + zo * p.sc_o + zi * p.sc_i + m * p.ldc + n0;
  if (cnt == 4 && p.vec_store) {
    if (sizeof(TO) == 4) {
      *reinterpret_cast<float4*>(c) = make_float4(v[0], v[1], v[2], v[3]);
    } else {
      uint2 w;
      w.x = (uint32_t)f2bf(v[0]) | ((uint32_t)f2bf(v[1]) << 16);
      w.y = (uint32_t)f2bf(v[2]) | ((uint32_t)f2bf(v[3]) << 16);
      *reinterpret_cast<uint2*>(c) = w;
    }
  } else {
    for (int e = 0; e < cnt; ++e) Elem<TO>::store(c + e, v[e]);
  }
}

template <typename TO, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_mfma_kernel(GemmParams p) {
  constexpr int BK = 64;               // bf16 elements of K per tile (8 chunks of 16 B)
  constexpr int WM = BM / 2, WN = BN / 2;  // 2 x 2 waves
  constexpr int TM = WM / 16, TN = WN / 16;
  constexpr int A_CH = BM * BK / 8 / 256;  // 16-byte chunks per thread and tile
  constexpr int B_CH = BN * BK / 8 / 256;
  static_assert(A_CH >= 1 && B_CH >= 1, "tile too small for 256 threads");
  __shared__ __attribute__((aligned(16))) bf16_t As[2][BM * BK];
  __shared__ __attribute__((aligned(16))) bf16_t Bs[2][BN * BK];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t z = blockIdx.z;
  const int64_t zo = z / p.batch_inner, zi = z % p.batch_inner;
  const int tile = blockIdx.x;
  const int64_t m0 = (int64_t)(tile / p.tiles_n) * BM;
  const int64_t n0 = (int64_t)(tile % p.tiles_n) * BN;
  const bf16_t* A = (const bf16_t*)p.A + zo * p.sa_o + zi * p.sa_i;
  const bf16_t* B = (const bf16_t*)p.B + zo * p.sb_o + zi * p.sb_i;
  const int64_t M = p.M, N = p.N, K = p.K;

  uint4 ra[A_CH], rb[B_CH];
  auto load_tile = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int idx = i * 256 + tid, r = idx >> 3, c = idx & 7;
      const int64_t gm = min(m0 + r, M - 1);  // clamped rows are computed, never stored
      const int64_t gk = k0 + c * 8;
      ra[i] = gk < K ? *reinterpret_cast<const uint4*>(A + gm * p.lda + gk) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int idx = i * 256 + tid, r = idx >> 3, c = idx & 7;
      const int64_t gn = min(n0 + r, N - 1);
      const int64_t gk = k0 + c * 8;
      rb[i] = gk < K ? *reinterpret_cast<const uint4*>(B + gn * p.ldb + gk) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_tile = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_CH; ++i) {
      const int idx = i * 256 + tid, r = idx >> 3, c = idx & 7;
      *reinterpret_cast<uint4*>(&As[buf][r * BK + ((c ^ (r & 7)) << 3)]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_CH; ++i) {
      const int idx = i * 256 + tid, r = idx >> 3, c = idx & 7;
      *reinterpret_cast<uint4*>(&Bs[buf][r * BK + ((c ^ (r & 7)) << 3)]) = rb[i];
    }
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
  for (int kt = 0; kt < nk; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < nk) load_tile((int64_t)(kt + 1) * BK);
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      const int c = s * 4 + fc;
      bf16x8 af[TM], bfr[TN];
#pragma unroll
      for (int i = 0; i < TM; ++i) {
        const int r = wm * WM + i * 16 + fr;
        af[i] = *reinterpret_cast<const bf16x8*>(&As[cur][r * BK + ((c ^ (r & 7)) << 3)]);
      }
#pragma unroll
      for (int j = 0; j < TN; ++j) {
        const int r = wn * WN + j * 16 + fr;
        bfr[j] = *reinterpret_cast<const bf16x8*>(&Bs[cur][r * BK + ((c ^ (r & 7)) << 3)]);
      }
#pragma unroll
      for (int i = 0; i < TM; ++i)
#pragma unroll
        for (int j = 0; j < TN; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bfr[j], af[i], acc[i][j], 0, 0, 0);
    }
    if (kt + 1 < nk) store_tile(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int i = 0; i < TM; ++i)
#pragma unroll
    for (int j = 0; j < TN; ++j) {
      const int64_t m = m0 + wm * WM + i * 16 + fr;
      const int64_t n = n0 + wn * WN + j * 16 + 4 * fc;
      float v[4] = {acc[i][j][0], acc[i][j][1], acc[i][j][2], acc[i][j][3]};
      epilogue4<bf16_t, TO>(p, zo, zi, m, n, v);
    }
}

template <typename TI, typename TO>
__global__ __launch_bounds__(256) void gemm_simt_kernel(GemmParams p) {
  constexpr int BM = 64, BN = 64, BK = 16;
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
  float acc[4][4] = {};
  for (int64_t k0 = 0; k0 < p.K; k0 += BK) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const int idx = e * 256 + tid;
      {
        const int r = idx / BK, kk = idx % BK;
        const int64_t gm = m0 + r, gk = k0 + kk;
        As[kk][r] = (gm < p.M && gk < p.K) ? Elem<TI>::load(A + gm * p.lda + gk) : 0.f;
      }
      if (p.b_kn) {
        const int kk = idx / BN, c = idx % BN;
        const int64_t gn = n0 + c, gk = k0 + kk;
        Bs[kk][c] = (gn < p.N && gk < p.K) ? Elem<TI>::load(B + gk * p.ldb + gn) : 0.f;
      } else {
        const int c = idx / BK, kk = idx % BK;
        const int64_t gn = n0 + c, gk = k0 + kk;
        Bs[kk][c] = (gn < p.N && gk < p.K) ? Elem<TI>::load(B + gn * p.ldb + gk) : 0.f;
      }
    }
    __syncthreads();
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
#pragma unroll
  for (int i = 0; i < 4; ++i) epilogue4<TI, TO>(p, zo, zi, m0 + ty * 4 + i, n0 + tx * 4, acc[i]);
}

static inline bool al16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

}  // namespace tl

using namespace tl;

extern "C" int tl_gemm(tl_ctx* ctx, const tl_gemm_desc* d) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(d, "null descriptor");
  TL_REQUIRE(d->M > 0 && d->N > 0 && d->K > 0, "GEMM sizes must be positive (M=%lld N=%lld K=%lld)",
             (long long)d->M, (long long)d->N, (long long)d->K);
  TL_REQUIRE(d->A && d->B, "null operand");
  TL_REQUIRE(dtype_is_float(d->dtype_in) && dtype_is_float(d->dtype_out), "GEMM dtypes must be fp32 or bf16");
  TL_REQUIRE(d->b_layout == TL_B_NK || d->b_layout == TL_B_KN, "bad b_layout %d", d->b_layout);
  TL_REQUIRE(d->act == TL_ACT_NONE || d->act == TL_ACT_GELU || d->act == TL_ACT_SILU, "bad activation");
  TL_REQUIRE(d->divisor != 0.f, "divisor must be non-zero");
  const int64_t batch = d->batch <= 0 ? 1 : d->batch;
  const int64_t binner = d->batch_inner <= 0 ? 1 : d->batch_inner;
  TL_REQUIRE(batch <= 65535, "batch %lld exceeds 65535", (long long)batch);
  TL_REQUIRE(d->lda >= d->K, "lda < K");
  TL_REQUIRE(d->b_layout == TL_B_NK ? d->ldb >= d->K : d->ldb >= d->N, "ldb too small");
  const bool qkv = d->epilogue == TL_EPI_QKV_SPLIT;
  TL_REQUIRE(d->epilogue == TL_EPI_STORE || qkv, "bad epilogue %d", d->epilogue);
  if (qkv) {
    TL_REQUIRE(d->q && d->k && d->vt, "QKV split needs q, k and vt");
    TL_REQUIRE(batch == 1 && !d->residual, "QKV split is unbatched and has no residual");
    TL_REQUIRE(d->seq_len > 0 && d->M % d->seq_len == 0, "M must be a multiple of seq_len");
    TL_REQUIRE(d->head_dim > 0 && d->n_heads_q > 0 && d->n_heads_kv > 0 &&
                   d->n_heads_q % d->n_heads_kv == 0,
               "bad head configuration");
    TL_REQUIRE(d->N == (d->n_heads_q + 2 * d->n_heads_kv) * d->head_dim, "N != (Hq + 2 Hkv) * Dh");
  } else {
    TL_REQUIRE(d->C, "null output");
    TL_REQUIRE(d->ldc >= d->N, "ldc < N");
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
  p.T = d->seq_len; p.Hq = d->n_heads_q; p.Hkv = d->n_heads_kv; p.Dh = d->head_dim;
  const size_t eo = dtype_size(d->dtype_out);
  p.vec_store = !qkv && d->ldc % 4 == 0 && ((uintptr_t)d->C % (4 * eo)) == 0 &&
                d->sc_o % 4 == 0 && d->sc_i % 4 == 0;

  // The MFMA kernel streams 16-byte rows of A and Bt: K-contiguous, 8-element aligned.
  const bool mfma = d->dtype_in == TL_BF16 && d->b_layout == TL_B_NK && d->K % 8 == 0 &&
                    d->lda % 8 == 0 && d->ldb % 8 == 0 && d->sa_o % 8 == 0 &&
                    d->sa_i % 8 == 0 && d->sb_o % 8 == 0 && d->sb_i % 8 == 0 && al16(d->A) &&
                    al16(d->B);
  const double es_in = (double)dtype_size(d->dtype_in);
  const double flops = 2.0 * d->M * d->N * d->K * batch;
  const double bytes = batch * (es_in * ((double)d->M * d->K + (double)d->N * d->K) +
                                (double)eo * d->M * d->N * (d->residual ? 2 : 1));
  const int family = mfma ? d->family : TL_KF_GEMM_SIMT;
  TL_REQUIRE(family >= 0 && family < TL_KF_COUNT, "bad kernel family");
  LaunchScope ls(ctx, family, flops, bytes);
  const bool f32out = d->dtype_out == TL_F32;
  if (mfma) {
    // 128x128 tiles, or 64x64 when 128x128 leaves most of the 256 CUs idle.
    const int64_t t128 = ((d->M + 127) / 128) * ((d->N + 127) / 128) * batch;
    const bool small = t128 < 2LL * (ctx->num_cus > 0 ? ctx->num_cus : 256);
    const int bm = small ? 64 : 128, bn = bm;
    p.tiles_m = (int)((d->M + bm - 1) / bm);
    p.tiles_n = (int)((d->N + bn - 1) / bn);
    TL_REQUIRE((int64_t)p.tiles_m * p.tiles_n < 0x7fffffff, "too many tiles");
    dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
    if (small) {
      if (f32out) gemm_mfma_kernel<float, 64, 64><<<grid, 256, 0, ctx->stream>>>(p);
      else gemm_mfma_kernel<bf16_t, 64, 64><<<grid, 256, 0, ctx->stream>>>(p);
    } else {
      if (f32out) gemm_mfma_kernel<float, 128, 128><<<grid, 256, 0, ctx->stream>>>(p);
      else gemm_mfma_kernel<bf16_t, 128, 128><<<grid, 256, 0, ctx->stream>>>(p);
    }
    return ls.finish("gemm_mfma");
  }
  p.tiles_m = (int)((d->M + 63) / 64);
  p.tiles_n = (int)((d->N + 63) / 64);
  TL_REQUIRE((int64_t)p.tiles_m * p.tiles_n < 0x7fffffff, "too many tiles");
  dim3 grid((unsigned)(p.tiles_m * p.tiles_n), 1, (unsigned)batch);
  if (d->dtype_in == TL_F32) {
    if (f32out) gemm_simt_kernel<float, float><<<grid, 256, 0, ctx->stream>>>(p);
    else gemm_simt_kernel<float, bf16_t><<<grid, 256, 0, ctx->stream>>>(p);
  } else {
    if (f32out) gemm_simt_kernel<bf16_t, float><<<grid, 256, 0, ctx->stream>>>(p);
    else gemm_simt_kernel<bf16_t, bf16_t><<<grid, 256, 0, ctx->stream>>>(p);
  }
  return ls.finish("gemm_simt");
}
