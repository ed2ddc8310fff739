// Fused causal attention: scores, mask, online softmax, P.V and the head merge in one
// kernel (replaces the reference's materialised [B, H, T, T] path, layers.py:293-304).
//
// Layout: q [B, Hq, Tq, D], k [B, Hkv, Tk, D], vt [B, Hkv, D, Tk] (bf16, as the QKV GEMM's
// split epilogue writes them); out [B, Tq, Hq*D] with row pitch ld_out. Query head h reads
// kv head h / (Hq / Hkv).
//
// One workgroup = 4 wavefronts = 64 query rows of one (batch, head); each wave owns 16
// rows. Key/value chunks of 64 positions are double-buffered in LDS and shared by the 4
// waves; causal blocks stop at the last chunk their rows can see. Per chunk a wave runs
//   S^T = K Q^T  on the MFMA (v_mfma_f32_16x16x32_bf16): lane l holds the scores of query
//                row l % 16 at 4 consecutive key positions per 16-key tile,
//   online softmax in fp32 on those registers (row max / sum across the 4 lanes that
//                share a row: two xor shuffles),
//   O^T += V^T P^T on the MFMA, with P converted to bf16 in place: a lane's 8 probabilities
//                (two 4-key runs) are its B operand as they stand, and the V^T fragment is
//                read with the same key permutation, so no data moves between lanes.
// The final O / l is written as 4 consecutive head-dim values per lane.
#include "tl_internal.hpp"

namespace tl {

struct AttnParams {
  const bf16_t* q;
  const bf16_t* k;
  const bf16_t* vt;
  bf16_t* out;
  int Hq, Hkv, Tq, Tk, Lk;  // Lk: key/value capacity (row pitch of vt, rows of k)
  int64_t ld_out;
  int64_t offset;
  float scale_log2;  // log2(e) / divisor
  int causal;
};

template <int D>
__global__ __launch_bounds__(256) void attention_fwd_kernel(AttnParams p) {
  constexpr int BKV = 64;
  constexpr int KCH = D / 8;          // 16-byte chunks per K row
  constexpr int KSW = KCH >= 8 ? 7 : KCH - 1;
  constexpr int DT = D / 16;          // 16-row d tiles of the output
  constexpr int KS = D / 32;          // 32-wide k steps of Q.K
  constexpr int K_LOADS = BKV * KCH / 256;  // chunks per thread per K tile
  constexpr int V_LOADS = D * 8 / 256;      // V^T tile: D rows x 8 chunks
  static_assert(K_LOADS >= 1 && V_LOADS >= 1, "head_dim too small");
  __shared__ __attribute__((aligned(16))) bf16_t Ks[2][BKV * D];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[2][D * BKV];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, fg = lane >> 4;
  const int bh = blockIdx.y;
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const int nqb = (p.Tq + 63) / 64;
  const int qb = nqb - 1 - (int)blockIdx.x;  // heaviest causal blocks first
  const int q0 = qb * 64 + wave * 16;
  const bf16_t* qh = p.q + ((int64_t)(b * p.Hq + h) * p.Tq) * D;
  const bf16_t* kh = p.k + ((int64_t)(b * p.Hkv + hk) * p.Lk) * D;
  const bf16_t* vh = p.vt + ((int64_t)(b * p.Hkv + hk) * D) * p.Lk;

  // Q fragments (B operand of S^T): lane holds Q[q0 + fr][32 s + 8 fg .. +7]
  bf16x8 qf[KS];
  {
    const int qi = min(q0 + fr, p.Tq - 1);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[s] = *reinterpret_cast<const bf16x8*>(qh + (int64_t)qi * D + 32 * s + 8 * fg);
  }

  // kv range this block needs
  const int q_last = min(qb * 64 + 63, p.Tq - 1);
  int kv_end = p.Tk;
  if (p.causal) kv_end = (int)min((int64_t)p.Tk, (int64_t)q_last + p.offset + 1);
  const int nchunks = (kv_end + BKV - 1) / BKV;

  uint4 rk[K_LOADS], rv[V_LOADS];
  auto load_chunk_regs = [&](int kv0) {
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int idx = i * 256 + tid, r = idx / KCH, c = idx % KCH;
      const int kv = kv0 + r;
      rk[i] = kv < p.Tk ? *reinterpret_cast<const uint4*>(kh + (int64_t)kv * D + c * 8) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < V_LOADS; ++i) {
      const int idx = i * 256 + tid, r = idx >> 3, c = idx & 7;
      // Lk % 8 == 0, so a chunk that starts below Tk lies inside the row; its keys past Tk
      // get probability 0 (their values must be finite)
      const int kv = kv0 + c * 8;
      rv[i] = kv < p.Tk ? *reinterpret_cast<const uint4*>(vh + (int64_t)r * p.Lk + kv) : make_uint4(0, 0, 0, 0);
    }
  };
  auto store_chunk_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int idx = i * 256 + tid, r = idx / KCH, c = idx % KCH;
      *reinterpret_cast<uint4*>(&Ks[buf][r * D + ((c ^ (r & KSW)) << 3)]) = rk[i];
    }
#pragma unroll
    for (int i = 0; i < V_LOADS; ++i) {
      const int idx = i * 256 + tid, r = idx >> 3, c = idx & 7;
      *reinterpret_cast<uint4*>(&Vs[buf][r * BKV + ((c ^ (r & 7)) << 3)]) = rv[i];
    }
  };

  f32x4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -INFINITY, l_run = 0.f;
  const int qpos = q0 + fr;  // this lane's query row (position qpos + offset)

  load_chunk_regs(0);
  store_chunk_lds(0);
  __syncthreads();
  for (int ch = 0; ch < nchunks; ++ch) {
    const int cur = ch & 1;
    const int kv0 = ch * BKV;
    if (ch + 1 < nchunks) load_chunk_regs(kv0 + BKV);

    // S^T for 4 key tiles of 16
    f32x4 s[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int r = j * 16 + fr;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int c = ks * 4 + fg;
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&Ks[cur][r * D + ((c ^ (r & KSW)) << 3)]);
        s[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], s[j], 0, 0, 0);
      }
    }
    // scale, mask, running max
    float mx = -INFINITY;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const int kv = kv0 + j * 16 + 4 * fg + v;
        const bool ok = kv < p.Tk && (!p.causal || (int64_t)kv <= (int64_t)qpos + p.offset);
        const float x = ok ? s[j][v] * p.scale_log2 : -INFINITY;
        s[j][v] = x;
        mx = fmaxf(mx, x);
      }
    mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
    mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
    const float m_new = fmaxf(m_run, mx);
    const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
    float rs = 0.f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        const float e = __builtin_amdgcn_exp2f(s[j][v] - m_new);
        s[j][v] = e;
        rs += e;
      }
    rs += __shfl_xor(rs, 16, 64);
    rs += __shfl_xor(rs, 32, 64);
    l_run = l_run * alpha + rs;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int v = 0; v < 4; ++v) o[t][v] *= alpha;

    // O^T += V^T P^T over two 32-key halves
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
      bf16x8 pf;
#pragma unroll
      for (int v = 0; v < 4; ++v) {
        pf[v] = (__bf16)s[2 * c2][v];
        pf[4 + v] = (__bf16)s[2 * c2 + 1][v];
      }
      // keys of item i: 32 c2 + 4 fg + i (i < 4) and 32 c2 + 16 + 4 fg + (i - 4)
      const int ka = 32 * c2 + 4 * fg, kb = ka + 16;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int r = t * 16 + fr;
        const bf16_t* row = &Vs[cur][r * BKV];
        const int ca = ka >> 3, cb = kb >> 3;
        const uint2 va = *reinterpret_cast<const uint2*>(row + ((ca ^ (r & 7)) << 3) + (ka & 7));
        const uint2 vb = *reinterpret_cast<const uint2*>(row + ((cb ^ (r & 7)) << 3) + (kb & 7));
        const uint4 vv = make_uint4(va.x, va.y, vb.x, vb.y);
        const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
        o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o[t], 0, 0, 0);
      }
    }

    if (ch + 1 < nchunks) store_chunk_lds(cur ^ 1);
    __syncthreads();
  }

  if (qpos < p.Tq) {
    const float inv = 1.0f / l_run;
    bf16_t* orow = p.out + ((int64_t)b * p.Tq + qpos) * p.ld_out + (int64_t)h * D;
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      uint2 w;
      w.x = (uint32_t)f2bf(o[t][0] * inv) | ((uint32_t)f2bf(o[t][1] * inv) << 16);
      w.y = (uint32_t)f2bf(o[t][2] * inv) | ((uint32_t)f2bf(o[t][3] * inv) << 16);
      *reinterpret_cast<uint2*>(orow + t * 16 + 4 * fg) = w;
    }
  }
}

}  // namespace tl

using namespace tl;

extern "C" int tl_attention_fwd(tl_ctx* ctx, const void* q, const void* k, const void* vt,
                                void* out, int64_t batch, int64_t n_heads_q, int64_t n_heads_kv,
                                int64_t seq_q, int64_t seq_k, int64_t head_dim, int64_t ld_out,
                                int64_t offset, float divisor, int32_t causal,
                                int64_t kv_capacity, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  TL_REQUIRE(q && k && vt && out, "null pointer");
  TL_REQUIRE(batch > 0 && n_heads_q > 0 && n_heads_kv > 0 && n_heads_q % n_heads_kv == 0,
             "bad batch/head configuration");
  TL_REQUIRE(seq_q > 0 && seq_k > 0 && seq_q < (1 << 30) && seq_k < (1 << 30), "bad sequence lengths");
  TL_REQUIRE(ld_out >= n_heads_q * head_dim, "ld_out < heads * head_dim");
  TL_REQUIRE(divisor > 0.f, "divisor must be positive");
  TL_REQUIRE(!causal || offset >= 0, "causal attention needs offset >= 0");
  TL_REQUIRE(batch * n_heads_q <= 65535, "batch * heads exceeds 65535");
  if (dtype != TL_BF16)
    return fail(TL_ERR_UNSUPPORTED, "fused attention is implemented for bf16 only");
  if (!(head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256))
    return fail(TL_ERR_UNSUPPORTED, "fused attention supports head_dim 32, 64, 128, 256");
  const int64_t cap = kv_capacity > 0 ? kv_capacity : seq_k;
  TL_REQUIRE(seq_k <= cap && cap < (1 << 30), "seq_k exceeds kv_capacity");
  if (cap % 8 != 0 || ld_out % 4 != 0)
    return fail(TL_ERR_UNSUPPORTED, "fused attention needs kv_capacity %% 8 == 0 and ld_out %% 4 == 0");
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)vt) & 15u || ((uintptr_t)out & 7u))
    return fail(TL_ERR_UNSUPPORTED, "fused attention needs 16-byte aligned q, k, vt");
  AttnParams p;
  p.q = (const bf16_t*)q; p.k = (const bf16_t*)k; p.vt = (const bf16_t*)vt; p.out = (bf16_t*)out;
  p.Hq = (int)n_heads_q; p.Hkv = (int)n_heads_kv; p.Tq = (int)seq_q; p.Tk = (int)seq_k;
  p.Lk = (int)cap;
  p.ld_out = ld_out; p.offset = offset; p.causal = causal ? 1 : 0;
  p.scale_log2 = 1.4426950408889634f / divisor;
  // algorithmic work: causal keeps sum over rows of min(Tk, t + offset + 1) keys
  double kept = 0;
  for (int64_t t = 0; t < seq_q; ++t)
    kept += (double)(causal ? std::min<int64_t>(seq_k, t + offset + 1) : seq_k);
  const double bh = (double)batch * n_heads_q;
  const double flops = bh * kept * 4.0 * head_dim;
  const double bytes = 2.0 * (bh * seq_q * head_dim * 2 + (double)batch * n_heads_kv * seq_k * head_dim * 2);
  LaunchScope ls(ctx, TL_KF_ATTENTION, flops, bytes);
  dim3 grid((unsigned)((seq_q + 63) / 64), (unsigned)(batch * n_heads_q));
  switch (head_dim) {
    case 32: attention_fwd_kernel<32><<<grid, 256, 0, ctx->stream>>>(p); break;
    case 64: attention_fwd_kernel<64><<<grid, 256, 0, ctx->stream>>>(p); break;
    case 128: attention_fwd_kernel<128><<<grid, 256, 0, ctx->stream>>>(p); break;
    default: attention_fwd_kernel<256><<<grid, 256, 0, ctx->stream>>>(p); break;
  }
  return ls.finish("attention_fwd");
}
