// Fused causal attention: scores, mask, online softmax, P.V and the head merge in one
// kernel (replaces the reference's materialised [B, H, T, T] path, layers.py:293-304).
//
// Layout: q [B, Hq, Tq, D], k [B, Hkv, Lk, D], vt [B, Hkv, D, Lk] (bf16, as the QKV GEMM's
// split epilogue writes them; the first Tk of the Lk positions are valid, Lk % 8 == 0);
// out [B, Tq, Hq*D] with row pitch ld_out. Query head h reads kv head h / (Hq / Hkv).
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
#include <mutex>

#include "tl_internal.hpp"

namespace tl {

// Keep the first n (1..7) bf16 values of an 8-value chunk and zero the rest: value rows
// past the last valid key.
__device__ __forceinline__ uint4 keep_first(uint4 v, int n) {
  uint32_t w[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if (2 * i >= n) w[i] = 0;
    else if (2 * i + 1 >= n) w[i] &= 0xffffu;
  }
  return make_uint4(w[0], w[1], w[2], w[3]);
}

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
  // decode with a device position: when set, query t sits at *pos_dev + t and keys
  // 0 .. *pos_dev + Tq - 1 (at most Lk) are valid; Tk and offset are read from it at run time
  const int64_t* pos_dev;
  // decode only: the rotate-half RoPE table [2, Tq, D/2] (cos, sin) of positions offset ..
  // offset + Tq - 1. When set, the decode kernel rotates the queries and this call's new
  // cache keys (positions offset ..) itself and writes the rotated keys back to the cache.
  const float* rope;
  // wide kernel, causal: CUs per round of the resident grid for its balanced block order
  // (0: heaviest first)
  int fold;
};

// V^T rows of a 64-key chunk in LDS (the long-sequence kernels): the P.V operand of lane
// group fg in 32-key half c2 is keys 32 c2 + 4 fg .. +3 and 32 c2 + 16 + 4 fg .. +3, so
// within each half the 4-key groups are stored in the order 0, 4, 1, 5, 2, 6, 3, 7 and a
// lane's 8 keys are one 16-byte piece, read straight into the MFMA operand. 16-byte pieces
// are XOR-swizzled by row (r & 7) against bank conflicts. Offsets in bf16 elements.
__device__ __forceinline__ int vperm_piece(int c2, int fg, int r) {
  return (((c2 * 4 + fg) ^ (r & 7)) << 3);
}
// the 8-byte slot of 4-key group g4 (keys 4 g4 .. 4 g4 + 3 of the chunk) in row r
__device__ __forceinline__ int vperm_slot(int g4, int r) {
  const int c2 = g4 >> 3, lg = g4 & 7;
  const int slot = lg < 4 ? 2 * lg : 2 * (lg - 4) + 1;  // 8-byte slot within the half
  return vperm_piece(c2, slot >> 1, r) + ((slot & 1) << 2);
}

// The same order for V^T rows of 128 keys (the short-sequence kernel), pieces swizzled by
// (r & 15).
__device__ __forceinline__ int vperm_piece16(int c2, int fg, int r) {
  return (((c2 * 4 + fg) ^ (r & 15)) << 3);
}
__device__ __forceinline__ int vperm_slot16(int g4, int r) {
  const int c2 = g4 >> 3, lg = g4 & 7;
  const int slot = lg < 4 ? 2 * lg : 2 * (lg - 4) + 1;
  return vperm_piece16(c2, slot >> 1, r) + ((slot & 1) << 2);
}

//
// NW = 8 (head dims 128 and 256): 8 waves, 128 query rows per workgroup, two waves per SIMD.
// A wave's state (16 rows x D outputs, its query fragments, the next chunk's loads) fits the
// 256 VGPRs of two waves per SIMD, so while one wave waits on its LDS fragment reads or runs
// its softmax the other issues MFMAs; with NW = 4 the single wave per SIMD (the 128 KB of K
// and V^T chunks at D = 256 allow one workgroup per CU) runs those phases one after another.
template <int D, int NW = 4>
__global__ __launch_bounds__(64 * NW) void attention_fwd_kernel(AttnParams p) {
  constexpr int BKV = 64, NT = 64 * NW, RB = 16 * NW;
  constexpr int KCH = D / 8;          // 16-byte chunks per K row
  constexpr int KSW = KCH >= 8 ? 7 : KCH - 1;
  constexpr int DT = D / 16;          // 16-row d tiles of the output
  constexpr int KS = D / 32;          // 32-wide k steps of Q.K
  constexpr int K_LOADS = BKV * KCH / NT;  // chunks per thread per K tile
  constexpr int V_LOADS = D * 8 / NT;      // V^T tile: D rows x 8 chunks
  static_assert(K_LOADS >= 1 && V_LOADS >= 1, "head_dim too small");
  __shared__ __attribute__((aligned(16))) bf16_t Ks[2][BKV * D];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[2][D * BKV];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, fg = lane >> 4;
  const int bh = blockIdx.y;
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const int nqb = (p.Tq + RB - 1) / RB;
  // Under a causal mask query blocks are processed in pairs (nqb-1-x, x): the pair's chunk
  // counts sum to nqb + 1 for every x, so all workgroups carry the same work. Without a
  // mask every block costs the same and each workgroup takes one.
  const int x = (int)blockIdx.x;
  for (int pass = 0; pass < (p.causal ? 2 : 1); ++pass) {
    const int qb = pass == 0 ? nqb - 1 - x : x;
    if (pass == 1 && qb >= nqb - 1 - x) break;
    const int q0 = qb * RB + wave * 16;
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
    const int q_last = min(qb * RB + RB - 1, p.Tq - 1);
    int kv_end = p.Tk;
    if (p.causal) kv_end = (int)min((int64_t)p.Tk, (int64_t)q_last + p.offset + 1);
    const int nchunks = (kv_end + BKV - 1) / BKV;

    uint4 rk[K_LOADS], rv[V_LOADS];
    // Per-thread 32-bit offsets from a per-chunk uniform base (SGPR-based addressing).
    uint32_t k_off[K_LOADS], v_off[V_LOADS];
  #pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int idx = i * NT + tid;
      k_off[i] = (uint32_t)((idx / KCH) * D + (idx % KCH) * 8);
    }
  #pragma unroll
    for (int i = 0; i < V_LOADS; ++i) {
      const int idx = i * NT + tid;
      v_off[i] = (uint32_t)((idx >> 3) * p.Lk + (idx & 7) * 8);
    }
    auto load_chunk_regs = [&](int kv0) {
      const bf16_t* kc = kh + (int64_t)kv0 * D;
      const bf16_t* vc = vh + kv0;
      if (kv0 + BKV <= p.Tk) {  // whole chunk valid (uniform)
  #pragma unroll
        for (int i = 0; i < K_LOADS; ++i) rk[i] = *reinterpret_cast<const uint4*>(kc + k_off[i]);
  #pragma unroll
        for (int i = 0; i < V_LOADS; ++i) rv[i] = *reinterpret_cast<const uint4*>(vc + v_off[i]);
        return;
      }
  #pragma unroll
      for (int i = 0; i < K_LOADS; ++i) {
        const int kv = kv0 + (i * NT + tid) / KCH;
        rk[i] = kv < p.Tk ? *reinterpret_cast<const uint4*>(kc + k_off[i]) : make_uint4(0, 0, 0, 0);
      }
  #pragma unroll
      for (int i = 0; i < V_LOADS; ++i) {
        // Lk % 8 == 0, so a chunk that starts below Tk lies inside the row; its positions
        // past Tk (capacity padding, never written) are zeroed, since 0 * NaN would not be 0
        const int kv = kv0 + ((i * NT + tid) & 7) * 8;
        rv[i] = kv < p.Tk ? *reinterpret_cast<const uint4*>(vc + v_off[i]) : make_uint4(0, 0, 0, 0);
        if (kv < p.Tk && kv + 8 > p.Tk) rv[i] = keep_first(rv[i], p.Tk - kv);
      }
    };
    auto store_chunk_lds = [&](int buf) {
  #pragma unroll
      for (int i = 0; i < K_LOADS; ++i) {
        const int idx = i * NT + tid, r = idx / KCH, c = idx % KCH;
        *reinterpret_cast<uint4*>(&Ks[buf][r * D + ((c ^ (r & KSW)) << 3)]) = rk[i];
      }
  #pragma unroll
      for (int i = 0; i < V_LOADS; ++i) {
        const int idx = i * NT + tid, r = idx >> 3, c = idx & 7;
        bf16_t* row = &Vs[buf][r * BKV];
        *reinterpret_cast<uint2*>(row + vperm_slot(2 * c, r)) = make_uint2(rv[i].x, rv[i].y);
        *reinterpret_cast<uint2*>(row + vperm_slot(2 * c + 1, r)) = make_uint2(rv[i].z, rv[i].w);
      }
    };

    f32x4 o[DT];
  #pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    // m_run: the row's reference max (log2 units, the same in the 4 lanes of a row);
    // l_part: this lane's share of the row sum (its own key columns), reduced across the 4
    // lanes once after the last chunk
    float m_run = -INFINITY, l_part = 0.f;
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
        // two waves per SIMD: keep each key tile's fragment reads next to its MFMAs (reading
        // all 32 of a chunk ahead would hold 128 more registers than the budget has)
        if constexpr (NW == 8) __builtin_amdgcn_sched_barrier(0);
      }
      // mask (only chunks that cross this wave's causal diagonal or the key count need one:
      // the test is uniform across the wave), row max of the raw scores
      float mx = -INFINITY;
      const bool full = kv0 + BKV <= p.Tk &&
                        (!p.causal || (int64_t)(kv0 + BKV - 1) <= (int64_t)q0 + p.offset);
      if (full) {
  #pragma unroll
        for (int j = 0; j < 4; ++j)
  #pragma unroll
          for (int v = 0; v < 4; ++v) mx = fmaxf(mx, s[j][v]);
      } else {
        // key kv0 + 16 j + 4 fg + v is visible when 16 j + v <= lim (one per-lane limit)
        const int lim = (int)max(min(min((int64_t)p.Tk - 1, p.causal ? (int64_t)qpos + p.offset
                                                                    : (int64_t)p.Tk - 1) -
                                         kv0 - 4 * fg, (int64_t)64), (int64_t)-1);
  #pragma unroll
        for (int j = 0; j < 4; ++j)
  #pragma unroll
          for (int v = 0; v < 4; ++v) {
            s[j][v] = j * 16 + v <= lim ? s[j][v] : -INFINITY;
            mx = fmaxf(mx, s[j][v]);
          }
      }
      // Lazy rescaling: the reference max m_run (log2 units) moves only when a row's max
      // exceeds it by more than 8, so the unnormalised probabilities stay below 2^8 (exact
      // in fp32, full relative precision in bf16) and O and l are rescaled only then. A
      // lane's own max decides whether any row may grow; only then (the first visible chunk,
      // rarely after) is the row max taken across the row's 4 lanes, so the common chunk
      // needs no cross-lane exchange.
      if (__any(mx * p.scale_log2 > m_run + 8.0f)) {
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mxs = mx * p.scale_log2;
        const bool grow = mxs > m_run + 8.0f;  // the same in the row's 4 lanes
        const float m_new = grow ? mxs : m_run;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);  // 0 when m_run was -inf
        l_part *= alpha;
  #pragma unroll
        for (int t = 0; t < DT; ++t)
  #pragma unroll
          for (int v = 0; v < 4; ++v) o[t][v] *= alpha;
        m_run = m_new;
      }
      const float m_ref = m_run == -INFINITY ? 0.f : m_run;  // a row with no visible key yet
  #pragma unroll
      for (int j = 0; j < 4; ++j)
  #pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][v], p.scale_log2, -m_ref));
          s[j][v] = e;
          l_part += e;
        }

      // O^T += V^T P^T over two 32-key halves
  #pragma unroll
      for (int c2 = 0; c2 < 2; ++c2) {
        bf16x8 pf;
  #pragma unroll
        for (int v = 0; v < 4; ++v) {
          pf[v] = (__bf16)s[2 * c2][v];
          pf[4 + v] = (__bf16)s[2 * c2 + 1][v];
        }
        // keys of item i: 32 c2 + 4 fg + i (i < 4) and 32 c2 + 16 + 4 fg + (i - 4): one
        // 16-byte piece of the permuted V^T row (vperm_slot)
  #pragma unroll
        for (int t = 0; t < DT; ++t) {
          const int r = t * 16 + fr;
          const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&Vs[cur][r * BKV + vperm_piece(c2, fg, r)]);
          o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o[t], 0, 0, 0);
          if constexpr (NW == 8) {
            if (t % 4 == 3) __builtin_amdgcn_sched_barrier(0);
          }
        }
      }

      if (ch + 1 < nchunks) store_chunk_lds(cur ^ 1);
      __syncthreads();
    }

    float l_run = l_part + __shfl_xor(l_part, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
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
}

// Wide variant for sequences longer than 64 (D 32 or 64): each wave owns 32 query rows as
// two 16-row MFMA groups, so every K and V fragment read from LDS feeds two MFMAs, and a
// workgroup of 4 waves covers 128 query rows, so every 64-key chunk moved into LDS serves
// twice the rows.
// The per-wave chain (S^T = K Q^T, online softmax with lazy rescaling, O^T += V^T P^T, the
// same lane layouts and key permutation) is attention_fwd_kernel's, per group. Grid:
// (batch x heads, 128-row blocks); block y = 0 is the last (under a causal mask the
// heaviest) block of every head, so the heaviest blocks of all heads start first.
template <int D>
__global__ __launch_bounds__(256) void attention_fwd_wide_kernel(AttnParams p) {
  constexpr int BKV = 64, G = 2, RB = 128;
  constexpr int KCH = D / 8;
  constexpr int KSW = KCH >= 8 ? 7 : KCH - 1;
  constexpr int DT = D / 16;
  constexpr int KS = D / 32;
  constexpr int K_LOADS = BKV * KCH / 256;
  constexpr int V_LOADS = D * 8 / 256;
  static_assert(K_LOADS >= 1 && V_LOADS >= 1, "head_dim too small");
  __shared__ __attribute__((aligned(16))) bf16_t Ks[2][BKV * D];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[2][D * BKV];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // uniform: scalar mask branches
  const int fr = lane & 15, fg = lane >> 4;
  const int nqb = (p.Tq + RB - 1) / RB;
  // Block ranks run heaviest first: rank r is head r % nbh, query block nqb - 1 - r / nbh
  // (a causal block reads qb + 1 chunks of 128 keys). When the whole grid is resident at
  // once (p.fold = CUs), workgroups land breadth-first, so CU c holds dispatch positions c,
  // c + CUs, c + 2 CUs; every second round of CUs then takes its ranks in reverse, so each
  // CU pairs heavy blocks with light ones (GPT-2 B 8 T 1024: busiest CU 34 -> 30 chunk
  // units against a mean of 27). Otherwise blocks keep the heaviest-first order.
  const int nbh = (int)gridDim.x;
  const int pos = (int)blockIdx.y * nbh + (int)blockIdx.x;
  int r = pos;
  if (p.fold) {
    const int t = pos / p.fold, c = pos - t * p.fold;
    if (t & 1) r = t * p.fold + min(p.fold, nbh * nqb - t * p.fold) - 1 - c;
  }
  const int bh = r % nbh;
  const int qb = nqb - 1 - r / nbh;
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const int w0 = qb * RB + wave * 32;  // first row of this wave; group g starts at w0 + 16 g
  const int off = (int)p.offset;        // < 2^30 (host-checked)
  const bf16_t* qh = p.q + ((int64_t)(b * p.Hq + h) * p.Tq) * D;
  const bf16_t* kh = p.k + ((int64_t)(b * p.Hkv + hk) * p.Lk) * D;
  const bf16_t* vh = p.vt + ((int64_t)(b * p.Hkv + hk) * D) * p.Lk;

  bf16x8 qf[G][KS];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    const int qi = min(w0 + 16 * g + fr, p.Tq - 1);
#pragma unroll
    for (int s = 0; s < KS; ++s)
      qf[g][s] = *reinterpret_cast<const bf16x8*>(qh + (int64_t)qi * D + 32 * s + 8 * fg);
  }
  const int q_last = min(qb * RB + RB - 1, p.Tq - 1);
  int kv_end = p.Tk;
  if (p.causal) kv_end = (int)min((int64_t)p.Tk, (int64_t)q_last + p.offset + 1);
  const int nchunks = (kv_end + BKV - 1) / BKV;

  uint4 rk[K_LOADS], rv[V_LOADS];
  uint32_t k_off[K_LOADS], v_off[V_LOADS];
#pragma unroll
  for (int i = 0; i < K_LOADS; ++i) {
    const int idx = i * 256 + tid;
    k_off[i] = (uint32_t)((idx / KCH) * D + (idx % KCH) * 8);
  }
#pragma unroll
  for (int i = 0; i < V_LOADS; ++i) {
    const int idx = i * 256 + tid;
    v_off[i] = (uint32_t)((idx >> 3) * p.Lk + (idx & 7) * 8);
  }
  auto load_chunk_regs = [&](int kv0) {
    const bf16_t* kc = kh + (int64_t)kv0 * D;
    const bf16_t* vc = vh + kv0;
    if (kv0 + BKV <= p.Tk) {
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i) rk[i] = *reinterpret_cast<const uint4*>(kc + k_off[i]);
#pragma unroll
      for (int i = 0; i < V_LOADS; ++i) rv[i] = *reinterpret_cast<const uint4*>(vc + v_off[i]);
      return;
    }
#pragma unroll
    for (int i = 0; i < K_LOADS; ++i) {
      const int kv = kv0 + (i * 256 + tid) / KCH;
      rk[i] = kv < p.Tk ? *reinterpret_cast<const uint4*>(kc + k_off[i]) : make_uint4(0, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < V_LOADS; ++i) {
      const int kv = kv0 + ((i * 256 + tid) & 7) * 8;
      rv[i] = kv < p.Tk ? *reinterpret_cast<const uint4*>(vc + v_off[i]) : make_uint4(0, 0, 0, 0);
      if (kv < p.Tk && kv + 8 > p.Tk) rv[i] = keep_first(rv[i], p.Tk - kv);
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
      bf16_t* row = &Vs[buf][r * BKV];
      *reinterpret_cast<uint2*>(row + vperm_slot(2 * c, r)) = make_uint2(rv[i].x, rv[i].y);
      *reinterpret_cast<uint2*>(row + vperm_slot(2 * c + 1, r)) = make_uint2(rv[i].z, rv[i].w);
    }
  };

  f32x4 o[G][DT];
#pragma unroll
  for (int g = 0; g < G; ++g)
#pragma unroll
    for (int t = 0; t < DT; ++t) o[g][t] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run[G], l_part[G];
#pragma unroll
  for (int g = 0; g < G; ++g) {
    m_run[g] = -INFINITY;
    l_part[g] = 0.f;
  }

  load_chunk_regs(0);
  store_chunk_lds(0);
  __syncthreads();
  for (int ch = 0; ch < nchunks; ++ch) {
    const int cur = ch & 1;
    const int kv0 = ch * BKV;
    if (ch + 1 < nchunks) load_chunk_regs(kv0 + BKV);

    // S^T for 4 key tiles of 16, both row groups from each K fragment
    f32x4 s[G][4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
#pragma unroll
      for (int g = 0; g < G; ++g) s[g][j] = f32x4{0.f, 0.f, 0.f, 0.f};
      const int r = j * 16 + fr;
#pragma unroll
      for (int ks = 0; ks < KS; ++ks) {
        const int c = ks * 4 + fg;
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&Ks[cur][r * D + ((c ^ (r & KSW)) << 3)]);
#pragma unroll
        for (int g = 0; g < G; ++g)
          s[g][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[g][ks], s[g][j], 0, 0, 0);
      }
    }
    bf16x8 pf[G][2];
#pragma unroll
    for (int g = 0; g < G; ++g) {
      const int q0 = w0 + 16 * g, qpos = q0 + fr;
      float mx = -INFINITY;
      const bool full = kv0 + BKV <= p.Tk && (!p.causal || kv0 + BKV - 1 <= q0 + off);
      if (full) {
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) mx = fmaxf(mx, s[g][j][v]);
      } else {
        // key kv0 + 16 j + 4 fg + v is visible when 16 j + v <= lim: one per-lane limit, so
        // each element is a compare against an immediate (no per-element key index)
        const int lim = min(p.Tk - 1, p.causal ? qpos + off : p.Tk - 1) - kv0 - 4 * fg;
#pragma unroll
        for (int j = 0; j < 4; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            s[g][j][v] = j * 16 + v <= lim ? s[g][j][v] : -INFINITY;
            mx = fmaxf(mx, s[g][j][v]);
          }
      }
      // lazy rescaling, as in attention_fwd_kernel
      if (__any(mx * p.scale_log2 > m_run[g] + 8.0f)) {
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mxs = mx * p.scale_log2;
        const bool grow = mxs > m_run[g] + 8.0f;
        const float m_new = grow ? mxs : m_run[g];
        const float alpha = __builtin_amdgcn_exp2f(m_run[g] - m_new);
        l_part[g] *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int v = 0; v < 4; ++v) o[g][t][v] *= alpha;
        m_run[g] = m_new;
      }
      const float m_ref = m_run[g] == -INFINITY ? 0.f : m_run[g];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[g][j][v], p.scale_log2, -m_ref));
          s[g][j][v] = e;
          l_part[g] += e;
        }
#pragma unroll
      for (int c2 = 0; c2 < 2; ++c2)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          pf[g][c2][v] = (__bf16)s[g][2 * c2][v];
          pf[g][c2][4 + v] = (__bf16)s[g][2 * c2 + 1][v];
        }
    }

    // O^T += V^T P^T over two 32-key halves, both row groups from each V fragment: a lane's
    // 8 keys are one 16-byte piece of the permuted V^T row (vperm_slot)
#pragma unroll
    for (int c2 = 0; c2 < 2; ++c2) {
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int r = t * 16 + fr;
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&Vs[cur][r * BKV + vperm_piece(c2, fg, r)]);
#pragma unroll
        for (int g = 0; g < G; ++g)
          o[g][t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf[g][c2], o[g][t], 0, 0, 0);
      }
    }

    if (ch + 1 < nchunks) store_chunk_lds(cur ^ 1);
    __syncthreads();
  }

#pragma unroll
  for (int g = 0; g < G; ++g) {
    float l_run = l_part[g] + __shfl_xor(l_part[g], 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    const int qpos = w0 + 16 * g + fr;
    if (qpos < p.Tq) {
      const float inv = 1.0f / l_run;
      bf16_t* orow = p.out + ((int64_t)b * p.Tq + qpos) * p.ld_out + (int64_t)h * D;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        uint2 w;
        w.x = (uint32_t)f2bf(o[g][t][0] * inv) | ((uint32_t)f2bf(o[g][t][1] * inv) << 16);
        w.y = (uint32_t)f2bf(o[g][t][2] * inv) | ((uint32_t)f2bf(o[g][t][3] * inv) << 16);
        *reinterpret_cast<uint2*>(orow + t * 16 + 4 * fg) = w;
      }
    }
  }
}

// Rotate-half RoPE of 8 consecutive elements a (index d < D/2) and their partners b
// (index d + D/2) with the table values in registers (c[0], c[1]: the 8 cosines; c[2], c[3]:
// the 8 sines), in fp32 and rounded to bf16 as a separate RoPE pass would store them.
__device__ __forceinline__ void rope8v(bf16x8& a, bf16x8& b, const float4 (&c)[4]) {
  const float cv[8] = {c[0].x, c[0].y, c[0].z, c[0].w, c[1].x, c[1].y, c[1].z, c[1].w};
  const float sv[8] = {c[2].x, c[2].y, c[2].z, c[2].w, c[3].x, c[3].y, c[3].z, c[3].w};
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const float fa = (float)a[e], fb = (float)b[e];
    a[e] = (__bf16)(fa * cv[e] - fb * sv[e]);
    b[e] = (__bf16)(fb * cv[e] + fa * sv[e]);
  }
}

// Keep the first n of a run of 4 bf16 values (all of them for n >= 4, none for n <= 0),
// with selects rather than branches.
__device__ __forceinline__ uint2 keep_below(uint2 v, int n) {
  const uint32_t lo = n >= 2 ? 0xffffffffu : (n == 1 ? 0x0000ffffu : 0u);
  const uint32_t hi = n >= 4 ? 0xffffffffu : (n == 3 ? 0x0000ffffu : 0u);
  return make_uint2(v.x & lo, v.y & hi);
}

// ---------------------------------------------------------------------------------------
// Decode (split-KV) attention for a few query rows per kv head: the query rows that share a
// kv head (Hq / Hkv heads x Tq positions, at most 16) form one MFMA column block, so every
// key and value is read once per kv head rather than once per query head; the key range is
// split over many workgroups so the cache streams from HBM in parallel (flash-decoding,
// Dao et al. 2023). Each wave takes 16 J keys and keeps its scores, probabilities and P.V in
// registers with the same layouts as attention_fwd_kernel (K fragments and V^T fragments are
// read straight from global memory: each is used by one MFMA of one wave). The NW waves of a
// workgroup merge their (max, sum, O) in LDS and write one partial per workgroup;
// attention_combine_kernel rescales the partials by their maxima and writes O / l.
// ---------------------------------------------------------------------------------------
struct DecodeWs {
  float* o;   // [B*Hkv][nblk][16][D] unnormalised partial outputs
  float* ml;  // [B*Hkv][nblk][16][2] (max in log2 units, sum)
  int nblk;
};

template <int D, int NW, int J>
__global__ __launch_bounds__(64 * NW) void attention_decode_kernel(AttnParams p, DecodeWs w) {
  static_assert(J == 2 || J == 4, "16-key tiles per wave: 2 or 4");
  if (p.pos_dev) {  // the grid covers the capacity; blocks past the live keys write empty partials
    const int64_t pos = *p.pos_dev;
    p.offset = pos;
    p.Tk = (int)min(pos + (int64_t)p.Tq, (int64_t)p.Lk);
  }
  constexpr int KS = D / 32, DT = D / 16, KPW = 16 * J;
  __shared__ float sm[NW][16], sl[NW][16];
  __shared__ f32x4 so[NW][DT][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 15, grp = lane >> 4;
  const int bh = blockIdx.y;
  const int b = bh / p.Hkv, hk = bh - b * p.Hkv;
  const int g = p.Hq / p.Hkv;
  const int R = g * p.Tq;
  const bool rowok = col < R;
  const int jh = rowok ? col / p.Tq : 0, t = rowok ? col - jh * p.Tq : 0;
  const int64_t qpos = (int64_t)t + p.offset;
  const bf16x8 zero = {};

  // Every load below reads a clamped, in-bounds address unconditionally, and what lies past
  // the valid rows or keys is masked or zeroed afterwards. (With a condition on each load the
  // compiler gives each one its own exec-masked branch and waits for it inside, so the loads
  // completed one after another: 14.8 us per config-5 layer for 8.5 MB.)
  bf16x8 qf[KS];
  {
    const bf16_t* qrow = p.q + ((int64_t)(b * p.Hq + hk * g + jh) * p.Tq + t) * D + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = *reinterpret_cast<const bf16x8*>(qrow + 32 * ks);
  }
  // fused RoPE (D >= 64): element d = 32 ks + 8 grp + e of qf[ks] has its partner d + D/2 in
  // qf[ks + KS/2] of the same lane; the table row is loaded here, applied after the K and V
  // loads are issued
  constexpr int KH = KS / 2;
  float4 qcs[KH > 0 ? KH : 1][4];
  if constexpr (KH > 0) {
    if (p.rope) {
      const float* cs = p.rope + (int64_t)t * (D / 2) + 8 * grp;
      const float* sn = cs + (int64_t)p.Tq * (D / 2);
#pragma unroll
      for (int ks = 0; ks < KH; ++ks) {
        qcs[ks][0] = *reinterpret_cast<const float4*>(cs + 32 * ks);
        qcs[ks][1] = *reinterpret_cast<const float4*>(cs + 32 * ks + 4);
        qcs[ks][2] = *reinterpret_cast<const float4*>(sn + 32 * ks);
        qcs[ks][3] = *reinterpret_cast<const float4*>(sn + 32 * ks + 4);
      }
    }
  }
  const bf16_t* kh = p.k + (int64_t)bh * p.Lk * D;
  const bf16_t* vh = p.vt + (int64_t)bh * D * p.Lk;
  const int kc0 = (blockIdx.x * NW + wave) * KPW;

  // All of this wave's K and V^T fragments are requested up front (the V^T reads do not
  // depend on the softmax), so the wave waits for one memory round trip, not two. The
  // addresses are clamped to the cache capacity and do not depend on the live key count, so
  // with a device position the loads do not wait for it either; keys at or past Tk (cache
  // rows never written: any bits, NaN included) are masked out of the scores by a select and
  // their values zeroed below. A wave whose keys all lie past Tk reads a few such rows.
  bf16x8 kf[J][KS];
  // V^T rows in the key order of the P.V B operand: keys 32 hp + 4 grp + 0..3 and
  // 32 hp + 16 + 4 grp + 0..3 (values past Tk zeroed, since 0 * NaN would not be 0; the
  // capacity is a multiple of 8, so a 4-key run that starts inside it ends inside it)
  uint2 vfa[J / 2][DT], vfb[J / 2][DT];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    const int key = min(kc0 + 16 * j + col, p.Lk - 1);
    const bf16_t* krow = kh + (int64_t)key * D + 8 * grp;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) kf[j][ks] = *reinterpret_cast<const bf16x8*>(krow + 32 * ks);
  }
#pragma unroll
  for (int hp = 0; hp < J / 2; ++hp) {
    const int ka = min(kc0 + 32 * hp + 4 * grp, p.Lk - 4), kb = min(kc0 + 32 * hp + 16 + 4 * grp, p.Lk - 4);
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const bf16_t* vrow = vh + (int64_t)(dt * 16 + col) * p.Lk;
      vfa[hp][dt] = *reinterpret_cast<const uint2*>(vrow + ka);
      vfb[hp][dt] = *reinterpret_cast<const uint2*>(vrow + kb);
    }
  }
  if (!rowok) {
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) qf[ks] = zero;
  }
  if constexpr (KH > 0) {
    if (p.rope) {
#pragma unroll
      for (int ks = 0; ks < KH; ++ks) rope8v(qf[ks], qf[ks + KH], qcs[ks]);
    }
  }
  // zero the values of keys >= Tk (unrotated key index: keys 32 hp + 4 grp + i)
#pragma unroll
  for (int hp = 0; hp < J / 2; ++hp) {
    const int na = p.Tk - (kc0 + 32 * hp + 4 * grp), nb = na - 16;
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      vfa[hp][dt] = keep_below(vfa[hp][dt], na);
      vfb[hp][dt] = keep_below(vfb[hp][dt], nb);
    }
  }
  // fused RoPE of this call's new keys (positions offset .. offset + Tq - 1): the one lane
  // group holding such a key rotates it and writes it back to the cache for later steps
  if constexpr (KH > 0) {
    if (p.rope) {
#pragma unroll
      for (int j = 0; j < J; ++j) {
        const int key = kc0 + 16 * j + col;
        const int64_t tn = (int64_t)key - p.offset;
        if (key < p.Tk && tn >= 0 && tn < p.Tq) {
          const float* cs = p.rope + tn * (D / 2) + 8 * grp;
          const float* sn = cs + (int64_t)p.Tq * (D / 2);
          bf16_t* krow = const_cast<bf16_t*>(kh) + (int64_t)key * D + 8 * grp;
          // the whole table row first, then the rotations and stores (a load after a store
          // to the cache would wait for it); with one query position (a decode step) the new
          // key's row is table row 0, which every lane already holds for its query (qcs)
          float4 kcs[KH][4];
          if (p.Tq == 1) {
#pragma unroll
            for (int ks = 0; ks < KH; ++ks)
#pragma unroll
              for (int c = 0; c < 4; ++c) kcs[ks][c] = qcs[ks][c];
          } else {
#pragma unroll
            for (int ks = 0; ks < KH; ++ks) {
              kcs[ks][0] = *reinterpret_cast<const float4*>(cs + 32 * ks);
              kcs[ks][1] = *reinterpret_cast<const float4*>(cs + 32 * ks + 4);
              kcs[ks][2] = *reinterpret_cast<const float4*>(sn + 32 * ks);
              kcs[ks][3] = *reinterpret_cast<const float4*>(sn + 32 * ks + 4);
            }
          }
#pragma unroll
          for (int ks = 0; ks < KH; ++ks) {
            rope8v(kf[j][ks], kf[j][ks + KH], kcs[ks]);
            *reinterpret_cast<bf16x8*>(krow + 32 * ks) = kf[j][ks];
            *reinterpret_cast<bf16x8*>(krow + 32 * (ks + KH)) = kf[j][ks + KH];
          }
        }
      }
    }
  }

  // S^T = K Q^T for J tiles of 16 keys: lane holds keys kc0 + 16 j + 4 grp + i of row col
  f32x4 s[J];
#pragma unroll
  for (int j = 0; j < J; ++j) {
    s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      s[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf[j][ks], qf[ks], s[j], 0, 0, 0);
  }
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int key = kc0 + 16 * j + 4 * grp + i;
      const bool ok = rowok && key < p.Tk && (!p.causal || (int64_t)key <= qpos);
      const float x = ok ? s[j][i] * p.scale_log2 : -INFINITY;
      s[j][i] = x;
      mx = fmaxf(mx, x);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  float sum = 0.f;
#pragma unroll
  for (int j = 0; j < J; ++j)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float e = mx == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(s[j][i] - mx);
      s[j][i] = e;
      sum += e;
    }
  sum += __shfl_xor(sum, 16, 64);
  sum += __shfl_xor(sum, 32, 64);

  // O^T = V^T P^T: B operand = this lane's 8 probabilities (keys 32 hp + 4 grp + 0..3 and
  // 32 hp + 16 + 4 grp + 0..3), A operand = V^T rows read with the same key order
  f32x4 o[DT];
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) o[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int hp = 0; hp < J / 2; ++hp) {
    bf16x8 pf;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      pf[i] = (__bf16)s[2 * hp][i];
      pf[4 + i] = (__bf16)s[2 * hp + 1][i];
    }
#pragma unroll
    for (int dt = 0; dt < DT; ++dt) {
      const uint2 va = vfa[hp][dt], vb = vfb[hp][dt];
      const bf16x8 vf = __builtin_bit_cast(bf16x8, make_uint4(va.x, va.y, vb.x, vb.y));
      o[dt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o[dt], 0, 0, 0);
    }
  }

  // merge the 4 waves: rows col, head-dim 16 dt + 4 grp + i
  if (grp == 0) {
    sm[wave][col] = mx;
    sl[wave][col] = sum;
  }
#pragma unroll
  for (int dt = 0; dt < DT; ++dt) so[wave][dt][lane] = o[dt];
  __syncthreads();
  const int64_t slot = (int64_t)bh * w.nblk + blockIdx.x;
  for (int e = threadIdx.x; e < DT * 64; e += 64 * NW) {
    const int dt = e >> 6, ln = e & 63, r = ln & 15;
    if (r >= R) continue;
    float m = -INFINITY;
#pragma unroll
    for (int v = 0; v < NW; ++v) m = fmaxf(m, sm[v][r]);
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int v = 0; v < NW; ++v) {
      const float f = sm[v][r] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(sm[v][r] - m);
      acc += so[v][dt][ln] * f;
    }
    *reinterpret_cast<f32x4*>(w.o + (slot * 16 + r) * D + dt * 16 + 4 * (ln >> 4)) = acc;
  }
  if (threadIdx.x < 16) {
    const int r = threadIdx.x;
    float m = -INFINITY, l = 0.f;
#pragma unroll
    for (int v = 0; v < NW; ++v) m = fmaxf(m, sm[v][r]);
#pragma unroll
    for (int v = 0; v < NW; ++v)
      l += sm[v][r] == -INFINITY ? 0.f : sl[v][r] * __builtin_amdgcn_exp2f(sm[v][r] - m);
    w.ml[(slot * 16 + r) * 2] = m;
    w.ml[(slot * 16 + r) * 2 + 1] = l;
  }
}

// One workgroup per (query row, batch x kv head). Thread d requests its first PF partial
// outputs of head-dim d and the (max, sum) pair of partial d before anything else (none of
// these loads depends on another), so the kernel waits for one memory round trip; the
// maxima give the weights exp2(m_k - max), and the partials are summed with those weights.
template <int D>
__global__ __launch_bounds__(D < 64 ? 64 : D) void attention_combine_kernel(AttnParams p, DecodeWs w) {
  constexpr int NT = D < 64 ? 64 : D;  // whole waves, so the shuffles see only live lanes
  constexpr int NWV = NT / 64;
  constexpr int PF = 64;                // partials prefetched into registers
  __shared__ float wk[1024];
  __shared__ float red[NWV];
  __shared__ float stats[2];
  const int r = blockIdx.x, bh = blockIdx.y, d = threadIdx.x;
  const int b = bh / p.Hkv, hk = bh - b * p.Hkv;
  const int g = p.Hq / p.Hkv;
  const int jh = r / p.Tq, t = r - jh * p.Tq;
  const int nblk = w.nblk;
  const int64_t base = (int64_t)bh * nblk;
  const float* src = w.o + (base * 16 + r) * D + min(d, D - 1);
  float pre[PF];
#pragma unroll
  for (int u = 0; u < PF; ++u) pre[u] = src[(int64_t)min(u, nblk - 1) * 16 * D];
  const float2 ml0 = *reinterpret_cast<const float2*>(w.ml + ((base + min(d, nblk - 1)) * 16 + r) * 2);
  float m = d < nblk ? ml0.x : -INFINITY;
  for (int k = d + NT; k < nblk; k += NT) m = fmaxf(m, w.ml[((base + k) * 16 + r) * 2]);
  m = wave_max(m);
  if ((d & 63) == 0) red[d >> 6] = m;
  __syncthreads();
  if (d == 0) {
    float mm = red[0];
    for (int i = 1; i < NWV; ++i) mm = fmaxf(mm, red[i]);
    stats[0] = mm;
  }
  __syncthreads();
  m = stats[0];
  float l = 0.f;
  if (d < nblk) {
    const float f = ml0.x == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(ml0.x - m);
    wk[d] = f;
    l = ml0.y * f;
  }
  for (int k = d + NT; k < nblk; k += NT) {
    const float mk = w.ml[((base + k) * 16 + r) * 2];
    const float f = mk == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mk - m);
    wk[k] = f;
    l += w.ml[((base + k) * 16 + r) * 2 + 1] * f;
  }
  l = wave_sum(l);
  if ((d & 63) == 0) red[d >> 6] = l;
  __syncthreads();
  if (d == 0) {
    float ll = 0.f;
    for (int i = 0; i < NWV; ++i) ll += red[i];
    stats[1] = ll;
  }
  __syncthreads();
  if (d >= D) return;
  // partial k always accumulates into acc[k % 4], in increasing k, so the sum does not
  // depend on how many (empty, weight-0) partials follow the last live one
  float acc[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int u = 0; u < PF; ++u)
    if (u < nblk) acc[u & 3] += pre[u] * wk[u];
  int k = PF;
  for (; k + 4 <= nblk; k += 4) {
#pragma unroll
    for (int u = 0; u < 4; ++u) acc[u] += src[(int64_t)(k + u) * 16 * D] * wk[k + u];
  }
  for (; k < nblk; ++k) acc[k & 3] += src[(int64_t)k * 16 * D] * wk[k];
  const float o = (acc[0] + acc[1]) + (acc[2] + acc[3]);
  const int h = hk * g + jh;
  p.out[((int64_t)b * p.Tq + t) * p.ld_out + (int64_t)h * D + d] = f2bf(o / stats[1]);
}

// Scratch of tl_attention_fwd_noalloc (the decode partials): a file-scope array that every
// GPU the library runs on holds until the process ends. In host code `scratch` names a
// host-side stand-in, not a device address; its address on each device comes from
// hipGetSymbolAddress (attention_scratch_setup) and only that address reaches kernels.
constexpr size_t kNoallocScratchBytes = (size_t)16 << 20;
static __device__ __align__(256) unsigned char scratch[kNoallocScratchBytes];

// The turn order of each device's scratch: the context whose stream last launched kernels
// that use it. An eager call from another context first makes its own stream wait for that
// context's noalloc_done event (a device-side wait, the host does not block), so eager calls
// from different contexts on one GPU take the array in turn instead of overlapping.
struct ScratchTurn {
  std::mutex mu;
  const tl_ctx* last = nullptr;
};
static ScratchTurn g_scratch_turn[256];

int attention_scratch_setup(tl_ctx* ctx) {
  static std::mutex mu;
  static void* by_device[256] = {};
  if (ctx->device < 0 || ctx->device >= 256)
    return fail(TL_ERR_NO_DEVICE, "device index %d out of range for the scratch table", ctx->device);
  {
    std::lock_guard<std::mutex> lock(mu);
    if (!by_device[ctx->device]) {
      void* ptr = nullptr;
      const hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
      if (e != hipSuccess || !ptr)
        return fail(TL_ERR_HIP, "hipGetSymbolAddress(scratch) on device %d: %s", ctx->device,
                    hipGetErrorString(e));
      by_device[ctx->device] = ptr;
    }
  }
  ctx->noalloc_scratch = by_device[ctx->device];
  TL_CHECK_HIP(hipEventCreateWithFlags(&ctx->noalloc_done, hipEventDisableTiming));
  return TL_OK;
}

void attention_scratch_release(tl_ctx* ctx) {
  if (ctx->device >= 0 && ctx->device < 256) {
    ScratchTurn& turn = g_scratch_turn[ctx->device];
    std::lock_guard<std::mutex> lock(turn.mu);
    if (turn.last == ctx) turn.last = nullptr;
  }
  if (ctx->noalloc_done) (void)hipEventDestroy(ctx->noalloc_done);
  ctx->noalloc_done = nullptr;
}

// Short sequences (at most 128 queries and 128 keys, e.g. the ViT-S/4 encoder's 65): one
// workgroup per (batch, head) with one wave per 16 query rows, all keys and values of the
// head staged in LDS once, and the softmax taken over the whole row at once (no running
// maximum, no rescaling). Keys are covered in NKH 32-key halves, so 65 keys cost 96 rather
// than the two 64-key chunks (128 keys) and 128 query rows of the long-sequence kernels.
// Lane layouts, the S^T = K Q^T and O^T = V^T P^T products and the key order are
// attention_fwd_kernel's.
template <int D, int NKH>
__global__ __launch_bounds__(512) void attention_fwd_short_kernel(AttnParams p) {
  constexpr int NK = 32 * NKH, NKT = 2 * NKH;
  constexpr int KCH = D / 8;
  constexpr int KSW = KCH >= 8 ? 7 : KCH - 1;
  constexpr int DT = D / 16, KS = D / 32;
  constexpr int VCH = 16;  // 16-byte chunks per staged V^T row (128 keys)
  __shared__ __attribute__((aligned(16))) bf16_t Ks[NK * D];
  __shared__ __attribute__((aligned(16))) bf16_t Vs[D * VCH * 8];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int nt = blockDim.x;
  const int fr = lane & 15, fg = lane >> 4;
  const int bh = blockIdx.x;
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const bf16_t* qh = p.q + ((int64_t)(b * p.Hq + h) * p.Tq) * D;
  const bf16_t* kh = p.k + ((int64_t)(b * p.Hkv + hk) * p.Lk) * D;
  const bf16_t* vh = p.vt + ((int64_t)(b * p.Hkv + hk) * D) * p.Lk;

  // stage K [NK, D] and V^T [D, NK] (keys past Tk as zeros: 0 * NaN would not be 0)
  for (int idx = tid; idx < NK * KCH; idx += nt) {
    const int r = idx / KCH, c = idx - r * KCH;
    const uint4 v = r < p.Tk ? *reinterpret_cast<const uint4*>(kh + (int64_t)r * D + c * 8)
                             : make_uint4(0, 0, 0, 0);
    *reinterpret_cast<uint4*>(&Ks[r * D + ((c ^ (r & KSW)) << 3)]) = v;
  }
  for (int idx = tid; idx < D * (NK / 8); idx += nt) {
    const int r = idx / (NK / 8), c = idx - r * (NK / 8);
    const int kv = c * 8;
    uint4 v = kv < p.Tk ? *reinterpret_cast<const uint4*>(vh + (int64_t)r * p.Lk + kv)
                        : make_uint4(0, 0, 0, 0);
    if (kv < p.Tk && kv + 8 > p.Tk) v = keep_first(v, p.Tk - kv);
    bf16_t* row = &Vs[r * (VCH * 8)];
    *reinterpret_cast<uint2*>(row + vperm_slot16(2 * c, r)) = make_uint2(v.x, v.y);
    *reinterpret_cast<uint2*>(row + vperm_slot16(2 * c + 1, r)) = make_uint2(v.z, v.w);
  }
  const int q0 = wave * 16;
  bf16x8 qf[KS];
  {
    const int qi = min(q0 + fr, p.Tq - 1);
#pragma unroll
    for (int ks = 0; ks < KS; ++ks)
      qf[ks] = *reinterpret_cast<const bf16x8*>(qh + (int64_t)qi * D + 32 * ks + 8 * fg);
  }
  __syncthreads();

  f32x4 s[NKT];
#pragma unroll
  for (int j = 0; j < NKT; ++j) {
    s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    const int r = j * 16 + fr;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      const int c = ks * 4 + fg;
      const bf16x8 kf = *reinterpret_cast<const bf16x8*>(&Ks[r * D + ((c ^ (r & KSW)) << 3)]);
      s[j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(kf, qf[ks], s[j], 0, 0, 0);
    }
  }
  const int qpos = q0 + fr;
  float mx = -INFINITY;
  // key 16 j + 4 fg + v is visible when 16 j + v <= lim (one per-lane limit)
  const int lim = (int)max(min(min((int64_t)p.Tk - 1, p.causal ? (int64_t)qpos + p.offset
                                                              : (int64_t)p.Tk - 1) - 4 * fg,
                               (int64_t)16 * NKT), (int64_t)-1);
#pragma unroll
  for (int j = 0; j < NKT; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      s[j][v] = j * 16 + v <= lim ? s[j][v] * p.scale_log2 : -INFINITY;
      mx = fmaxf(mx, s[j][v]);
    }
  mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
  mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
  const float m_ref = mx == -INFINITY ? 0.f : mx;
  float l = 0.f;
#pragma unroll
  for (int j = 0; j < NKT; ++j)
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      const float e = __builtin_amdgcn_exp2f(s[j][v] - m_ref);
      s[j][v] = e;
      l += e;
    }
  l += __shfl_xor(l, 16, 64);
  l += __shfl_xor(l, 32, 64);

  f32x4 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c2 = 0; c2 < NKH; ++c2) {
    bf16x8 pf;
#pragma unroll
    for (int v = 0; v < 4; ++v) {
      pf[v] = (__bf16)s[2 * c2][v];
      pf[4 + v] = (__bf16)s[2 * c2 + 1][v];
    }
#pragma unroll
    for (int t = 0; t < DT; ++t) {
      const int r = t * 16 + fr;
      const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&Vs[r * (VCH * 8) + vperm_piece16(c2, fg, r)]);
      o[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vf, pf, o[t], 0, 0, 0);
    }
  }
  if (qpos < p.Tq) {
    const float inv = 1.0f / l;
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

// Resident wide-kernel workgroups per CU (register-limited: 3 at head dim 64), queried once;
// 0 if the query fails, which keeps the heaviest-first block order.
template <int D>
static int wide_blocks_per_cu() {
  static const int n = [] {
    int b = 0;
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&b, attention_fwd_wide_kernel<D>, 256, 0) != hipSuccess) {
      (void)hipGetLastError();
      return 0;
    }
    return b;
  }();
  return n;
}

template <int D>
static void launch_short(int nkh, dim3 grid, int threads, hipStream_t st, const AttnParams& p) {
  switch (nkh) {
    case 1: attention_fwd_short_kernel<D, 1><<<grid, threads, 0, st>>>(p); break;
    case 2: attention_fwd_short_kernel<D, 2><<<grid, threads, 0, st>>>(p); break;
    case 3: attention_fwd_short_kernel<D, 3><<<grid, threads, 0, st>>>(p); break;
    default: attention_fwd_short_kernel<D, 4><<<grid, threads, 0, st>>>(p); break;
  }
}

// fp32 attention (the reference's FLOAT_TYPE, backend.py:24; layers.py:286-304) on the
// fp32 matrix cores, v_mfma_f32_16x16x4f32: fp32 products and sums, so the scores, the
// softmax and P.V keep full fp32 precision. The structure is attention_fwd_kernel's: 4
// waves x 16 query rows, BKV-key chunks of K and V^T staged in LDS (registers -> LDS, double
// buffered), S^T = K Q^T so a lane holds 4 keys of one query row, online softmax with lazy
// rescaling, O^T += V^T P^T, causal query blocks paired so workgroups carry equal work.
// Chunks of 32 keys keep a workgroup's LDS at 32 KB (head dim 64), so three workgroups fit a
// CU and GPT-2's 768 paired blocks run as one round; 64-key chunks (64 KB) fit two, and the
// second half-round ran at one wave per SIMD.
// A 16x16x4 MFMA takes one element per lane per operand. Q.K sums over d in any order, so
// lane group fg covers the contiguous d range [fg D/4, (fg + 1) D/4) one d per MFMA (Q and K
// read as 16-byte chunks); P.V step u = (key tile j, v) takes key 16 j + 4 fg + v from lane
// group fg, which is exactly the probability that lane holds, and reads V^T[d][16 j + 4 fg
// .. + 3] as one 16-byte chunk. LDS rows are stored with their 16-byte chunks XOR-swizzled
// by row so the 16 rows of a fragment read hit distinct banks.
template <int D, int BKV>
__global__ __launch_bounds__(256) void attention_fwd_f32_kernel(AttnParams p) {
  constexpr int NJ = BKV / 16;       // 16-key tiles per chunk
  constexpr int VCH = BKV / 4;       // 16-byte chunks per V^T row
  constexpr int KCH = D / 4;          // 16-byte chunks per K row
  constexpr int KSW = KCH - 1;        // swizzle mask of a K row (KCH is a power of two)
  constexpr int DQ = D / 4;           // d values per lane group (one per MFMA)
  constexpr int DT = D / 16;          // 16-row d tiles of the output
  constexpr int K_LOADS = BKV * KCH / 256;
  constexpr int V_LOADS = D * VCH / 256;  // V^T chunk: D rows x VCH chunks
  static_assert(K_LOADS >= 1 && V_LOADS >= 1, "head_dim too small");
  __shared__ __attribute__((aligned(16))) float Ks[2][BKV * D];
  __shared__ __attribute__((aligned(16))) float Vs[2][D * BKV];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int fr = lane & 15, fg = lane >> 4;
  const int bh = blockIdx.y;
  const int b = bh / p.Hq, h = bh - b * p.Hq;
  const int hk = h / (p.Hq / p.Hkv);
  const int nqb = (p.Tq + 63) / 64;
  const int x = (int)blockIdx.x;
  const float* qg = reinterpret_cast<const float*>(p.q);
  const float* kg = reinterpret_cast<const float*>(p.k);
  const float* vg = reinterpret_cast<const float*>(p.vt);
  float* og = reinterpret_cast<float*>(p.out);
  for (int pass = 0; pass < (p.causal ? 2 : 1); ++pass) {
    const int qb = pass == 0 ? nqb - 1 - x : x;
    if (pass == 1 && qb >= nqb - 1 - x) break;
    const int q0 = qb * 64 + wave * 16;
    const float* qh = qg + ((int64_t)(b * p.Hq + h) * p.Tq) * D;
    const float* kh = kg + ((int64_t)(b * p.Hkv + hk) * p.Lk) * D;
    const float* vh = vg + ((int64_t)(b * p.Hkv + hk) * D) * p.Lk;

    // Q (second operand of S^T): lane holds Q[q0 + fr][fg DQ + s], s < DQ
    float qf[DQ];
    {
      const int qi = min(q0 + fr, p.Tq - 1);
#pragma unroll
      for (int c = 0; c < DQ / 4; ++c) {
        const f32x4 v = *reinterpret_cast<const f32x4*>(qh + (int64_t)qi * D + fg * DQ + 4 * c);
        qf[4 * c] = v[0]; qf[4 * c + 1] = v[1]; qf[4 * c + 2] = v[2]; qf[4 * c + 3] = v[3];
      }
    }
    const int q_last = min(qb * 64 + 63, p.Tq - 1);
    int kv_end = p.Tk;
    if (p.causal) kv_end = (int)min((int64_t)p.Tk, (int64_t)q_last + p.offset + 1);
    const int nchunks = (kv_end + BKV - 1) / BKV;

    f32x4 rk[K_LOADS], rv[V_LOADS];
    auto load_chunk_regs = [&](int kv0) {
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i) {
        const int idx = i * 256 + tid, r = idx / KCH, c = idx % KCH;
        const int kv = kv0 + r;
        rk[i] = kv < p.Tk ? *reinterpret_cast<const f32x4*>(kh + (int64_t)kv * D + 4 * c)
                          : f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int i = 0; i < V_LOADS; ++i) {
        // positions past Tk (capacity padding, never written) are zeroed: 0 * NaN is not 0
        const int idx = i * 256 + tid, r = idx / VCH, c = idx % VCH;
        const int kv = kv0 + 4 * c;
        f32x4 v = {0.f, 0.f, 0.f, 0.f};
        if (kv < p.Tk) {
          v = *reinterpret_cast<const f32x4*>(vh + (int64_t)r * p.Lk + kv);
#pragma unroll
          for (int e = 1; e < 4; ++e)
            if (kv + e >= p.Tk) v[e] = 0.f;
        }
        rv[i] = v;
      }
    };
    auto store_chunk_lds = [&](int buf) {
#pragma unroll
      for (int i = 0; i < K_LOADS; ++i) {
        const int idx = i * 256 + tid, r = idx / KCH, c = idx % KCH;
        *reinterpret_cast<f32x4*>(&Ks[buf][r * D + ((c ^ (r & KSW)) << 2)]) = rk[i];
      }
#pragma unroll
      for (int i = 0; i < V_LOADS; ++i) {
        const int idx = i * 256 + tid, r = idx / VCH, c = idx % VCH;
        *reinterpret_cast<f32x4*>(&Vs[buf][r * BKV + ((c ^ (r & (VCH - 1))) << 2)]) = rv[i];
      }
    };

    f32x4 o[DT];
#pragma unroll
    for (int t = 0; t < DT; ++t) o[t] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m_run = -INFINITY, l_part = 0.f;
    const int qpos = q0 + fr;

    load_chunk_regs(0);
    store_chunk_lds(0);
    __syncthreads();
    for (int ch = 0; ch < nchunks; ++ch) {
      const int cur = ch & 1;
      const int kv0 = ch * BKV;
      if (ch + 1 < nchunks) load_chunk_regs(kv0 + BKV);

      f32x4 s[NJ];
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        s[j] = f32x4{0.f, 0.f, 0.f, 0.f};
        const int r = j * 16 + fr;
#pragma unroll
        for (int c = 0; c < DQ / 4; ++c) {
          const int cc = fg * (DQ / 4) + c;
          const f32x4 kf = *reinterpret_cast<const f32x4*>(&Ks[cur][r * D + ((cc ^ (r & KSW)) << 2)]);
#pragma unroll
          for (int e = 0; e < 4; ++e)
            s[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(kf[e], qf[4 * c + e], s[j], 0, 0, 0);
        }
      }
      float mx = -INFINITY;
      const bool full = kv0 + BKV <= p.Tk &&
                        (!p.causal || (int64_t)(kv0 + BKV - 1) <= (int64_t)q0 + p.offset);
      if (full) {
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) mx = fmaxf(mx, s[j][v]);
      } else {
        // key kv0 + 16 j + 4 fg + v is visible when 16 j + v <= lim (one per-lane limit)
        const int lim = (int)max(min(min((int64_t)p.Tk - 1, p.causal ? (int64_t)qpos + p.offset
                                                                    : (int64_t)p.Tk - 1) -
                                         kv0 - 4 * fg, (int64_t)BKV), (int64_t)-1);
#pragma unroll
        for (int j = 0; j < NJ; ++j)
#pragma unroll
          for (int v = 0; v < 4; ++v) {
            s[j][v] = j * 16 + v <= lim ? s[j][v] : -INFINITY;
            mx = fmaxf(mx, s[j][v]);
          }
      }
      if (__any(mx * p.scale_log2 > m_run + 8.0f)) {
        mx = fmaxf(mx, __shfl_xor(mx, 16, 64));
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mxs = mx * p.scale_log2;
        const bool grow = mxs > m_run + 8.0f;
        const float m_new = grow ? mxs : m_run;
        const float alpha = __builtin_amdgcn_exp2f(m_run - m_new);
        l_part *= alpha;
#pragma unroll
        for (int t = 0; t < DT; ++t)
#pragma unroll
          for (int v = 0; v < 4; ++v) o[t][v] *= alpha;
        m_run = m_new;
      }
      const float m_ref = m_run == -INFINITY ? 0.f : m_run;
#pragma unroll
      for (int j = 0; j < NJ; ++j)
#pragma unroll
        for (int v = 0; v < 4; ++v) {
          const float e = __builtin_amdgcn_exp2f(__builtin_fmaf(s[j][v], p.scale_log2, -m_ref));
          s[j][v] = e;
          l_part += e;
        }
      // O^T += V^T P^T: step (j, v) takes key 16 j + 4 fg + v of lane group fg
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int r = t * 16 + fr;
#pragma unroll
        for (int j = 0; j < NJ; ++j) {
          const int cc = 4 * j + fg;
          const f32x4 vf = *reinterpret_cast<const f32x4*>(&Vs[cur][r * BKV + ((cc ^ (r & (VCH - 1))) << 2)]);
#pragma unroll
          for (int v = 0; v < 4; ++v)
            o[t] = __builtin_amdgcn_mfma_f32_16x16x4f32(vf[v], s[j][v], o[t], 0, 0, 0);
        }
      }
      if (ch + 1 < nchunks) store_chunk_lds(cur ^ 1);
      __syncthreads();
    }

    float l_run = l_part + __shfl_xor(l_part, 16, 64);
    l_run += __shfl_xor(l_run, 32, 64);
    if (qpos < p.Tq) {
      const float inv = 1.0f / l_run;
      float* orow = og + ((int64_t)b * p.Tq + qpos) * p.ld_out + (int64_t)h * D;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const f32x4 w = {o[t][0] * inv, o[t][1] * inv, o[t][2] * inv, o[t][3] * inv};
        *reinterpret_cast<f32x4*>(orow + t * 16 + 4 * fg) = w;
      }
    }
  }
}

// Decode split: waves per workgroup and 16-key tiles per wave. 2 waves x 32 keys was the
// fastest on an MI355X at the config-5 decode shape (B = 4, 2176 keys, D = 256) against
// (4, 4), (1, 4), (1, 2), (4, 2) and (2, 4): 12.0 us per layer with the combine, 13.5 us
// for 4 waves x 32 keys.
constexpr int kDecodeWaves = 2, kDecodeTiles = 2;

template <int D>
static void launch_decode(dim3 g1, dim3 g2, hipStream_t st, const AttnParams& p,
                          const DecodeWs& w) {
  attention_decode_kernel<D, kDecodeWaves, kDecodeTiles><<<g1, 64 * kDecodeWaves, 0, st>>>(p, w);
  attention_combine_kernel<D><<<g2, D < 64 ? 64 : D, 0, st>>>(p, w);
}

}  // namespace tl

using namespace tl;

// Both entry points. With noalloc the decode partials go to the static scratch array (its
// size is the limit) and the launch is kept out of the event profiler, so the call makes no
// allocation of any kind; otherwise they go to the context's grow-only workspace.
static int attention_fwd(tl_ctx* ctx, const void* q, const void* k, const void* vt, void* out,
                         int64_t batch, int64_t n_heads_q, int64_t n_heads_kv, int64_t seq_q,
                         int64_t seq_k, int64_t head_dim, int64_t ld_out, int64_t offset,
                         float divisor, int32_t causal, int64_t kv_capacity, int32_t dtype,
                         bool noalloc, const int64_t* pos_dev = nullptr,
                         const float* rope = nullptr) {
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
  if (dtype != TL_BF16 && dtype != TL_F32)
    return fail(TL_ERR_UNSUPPORTED, "fused attention takes bf16 or fp32");
  if (dtype == TL_F32 && !(head_dim == 32 || head_dim == 64 || head_dim == 128))
    return fail(TL_ERR_UNSUPPORTED, "fp32 fused attention supports head_dim 32, 64, 128");
  if (!(head_dim == 32 || head_dim == 64 || head_dim == 128 || head_dim == 256))
    return fail(TL_ERR_UNSUPPORTED, "fused attention supports head_dim 32, 64, 128, 256");
  const int64_t cap = kv_capacity > 0 ? kv_capacity : seq_k;
  TL_REQUIRE(seq_k <= cap && cap < (1 << 30), "seq_k exceeds kv_capacity");
  if (cap % 8 != 0 || ld_out % 4 != 0)
    return fail(TL_ERR_UNSUPPORTED, "fused attention needs kv_capacity %% 8 == 0 and ld_out %% 4 == 0");
  if (((uintptr_t)q | (uintptr_t)k | (uintptr_t)vt) & 15u || ((uintptr_t)out & 7u))
    return fail(TL_ERR_UNSUPPORTED, "fused attention needs 16-byte aligned q, k, vt");
  if (dtype == TL_F32 && (((uintptr_t)out & 15u) || (pos_dev || rope)))
    return fail(TL_ERR_UNSUPPORTED, "fp32 fused attention needs a 16-byte aligned output and "
                "takes no device position or fused RoPE");
  AttnParams p;
  p.q = (const bf16_t*)q; p.k = (const bf16_t*)k; p.vt = (const bf16_t*)vt; p.out = (bf16_t*)out;
  p.Hq = (int)n_heads_q; p.Hkv = (int)n_heads_kv; p.Tq = (int)seq_q; p.Tk = (int)seq_k;
  p.Lk = (int)cap;
  p.ld_out = ld_out; p.offset = offset; p.causal = causal ? 1 : 0;
  p.scale_log2 = 1.4426950408889634f / divisor;
  p.pos_dev = pos_dev;
  p.rope = rope;
  p.fold = 0;
  if (rope) {
    TL_REQUIRE(head_dim >= 64 && (n_heads_q / n_heads_kv) * seq_q <= 16 && causal && ((uintptr_t)rope & 15u) == 0,
               "fused RoPE is implemented for causal decode at head_dim >= 64 (16-byte aligned table)");
  }
  if (pos_dev) {
    TL_REQUIRE((uintptr_t)pos_dev % 8 == 0 && causal, "device positions need causal decode");
    if ((n_heads_q / n_heads_kv) * seq_q > 16)
      return fail(TL_ERR_UNSUPPORTED, "device positions are implemented for decode (at most 16 "
                  "query rows per kv head)");
  }
  // algorithmic work: causal keeps sum over rows of min(Tk, t + offset + 1) keys
  double kept = 0;
  for (int64_t t = 0; t < seq_q; ++t)
    kept += (double)(causal ? std::min<int64_t>(seq_k, t + offset + 1) : seq_k);
  const double bh = (double)batch * n_heads_q;
  const double flops = bh * kept * 4.0 * head_dim;
  const double bytes = 2.0 * (bh * seq_q * head_dim * 2 + (double)batch * n_heads_kv * seq_k * head_dim * 2);
  LaunchScope ls(ctx, noalloc ? -1 : TL_KF_ATTENTION, dtype == TL_F32 ? flops : flops,
                 dtype == TL_F32 ? 2.0 * bytes : bytes);
  if (dtype == TL_F32) {
    const int64_t nqb = (seq_q + 63) / 64;
    const dim3 grid((unsigned)(causal ? (nqb + 1) / 2 : nqb), (unsigned)(batch * n_heads_q));
    switch (head_dim) {
      case 32: attention_fwd_f32_kernel<32, 32><<<grid, 256, 0, ctx->stream>>>(p); break;
      case 64: attention_fwd_f32_kernel<64, 32><<<grid, 256, 0, ctx->stream>>>(p); break;
      default: attention_fwd_f32_kernel<128, 32><<<grid, 256, 0, ctx->stream>>>(p); break;
    }
    return ls.finish("attention_fwd_f32");
  }
  const int64_t rows_per_kv = (n_heads_q / n_heads_kv) * seq_q;
  if (rows_per_kv <= 16) {  // decode: split the keys over many small workgroups
    DecodeWs w;
    constexpr int nw = kDecodeWaves, jt = kDecodeTiles;
    // with a device position the key count is known only on the device: cover the capacity
    const int64_t keys = pos_dev ? cap : seq_k;
    w.nblk = (int)((keys + 16 * nw * jt - 1) / (16 * nw * jt));
    TL_REQUIRE(w.nblk <= 1024, "decode attention takes up to %d keys with this split",
               1024 * 16 * nw * jt);
    const int64_t slots = batch * n_heads_kv * w.nblk;
    TL_REQUIRE(batch * n_heads_kv <= 65535, "batch * kv heads exceeds 65535");
    void* ws;
    const size_t obytes = (size_t)slots * 16 * head_dim * sizeof(float);
    const size_t need = obytes + (size_t)slots * 16 * 2 * sizeof(float);
    // held from the wait on the previous user of the static scratch to the event recorded
    // after these kernels; not taken while the stream is being captured into a graph
    std::unique_lock<std::mutex> turn;
    if (noalloc) {
      if (need > kNoallocScratchBytes)
        return fail(TL_ERR_INVALID, "decode attention needs %zu bytes of partials; the "
                    "allocation-free entry point has %zu (tl_attention_fwd has no such limit)",
                    need, kNoallocScratchBytes);
      if (!ctx->noalloc_scratch || !ctx->noalloc_done)
        return fail(TL_ERR_HIP, "static scratch was not set up");
      ws = ctx->noalloc_scratch;
      hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
      TL_CHECK_HIP(hipStreamIsCapturing(ctx->stream, &cs));
      if (cs == hipStreamCaptureStatusNone) {
        ScratchTurn& t = g_scratch_turn[ctx->device];
        turn = std::unique_lock<std::mutex>(t.mu);
        if (t.last && t.last != ctx) TL_CHECK_HIP(hipStreamWaitEvent(ctx->stream, t.last->noalloc_done, 0));
      }
    } else {
      rc = workspace(ctx, need, &ws);
      if (rc) return rc;
    }
    w.o = (float*)ws;
    w.ml = (float*)((char*)ws + obytes);
    const dim3 g1((unsigned)w.nblk, (unsigned)(batch * n_heads_kv));
    const dim3 g2((unsigned)rows_per_kv, (unsigned)(batch * n_heads_kv));
    switch (head_dim) {
      case 32: launch_decode<32>(g1, g2, ctx->stream, p, w); break;
      case 64: launch_decode<64>(g1, g2, ctx->stream, p, w); break;
      case 128: launch_decode<128>(g1, g2, ctx->stream, p, w); break;
      default: launch_decode<256>(g1, g2, ctx->stream, p, w); break;
    }
    if (turn.owns_lock()) {
      TL_CHECK_HIP(hipEventRecord(ctx->noalloc_done, ctx->stream));
      g_scratch_turn[ctx->device].last = ctx;
    }
    return ls.finish("attention_decode");
  }
  // at most 128 queries and keys at head dim <= 128 (the ViT-S/4 encoder: 65): one workgroup
  // per (batch, head), the head's keys and values staged once, the softmax in one pass
  if (seq_q <= 128 && seq_k <= 128 && head_dim <= 128) {
    const int nkh = (int)((seq_k + 31) / 32);
    const int threads = (int)((seq_q + 15) / 16) * 64;
    const dim3 grid((unsigned)(batch * n_heads_q));
    switch (head_dim) {
      case 32: launch_short<32>(nkh, grid, threads, ctx->stream, p); break;
      case 64: launch_short<64>(nkh, grid, threads, ctx->stream, p); break;
      default: launch_short<128>(nkh, grid, threads, ctx->stream, p); break;
    }
    return ls.finish("attention_fwd_short");
  }
  // sequences longer than one 64-row block at head dim 32 / 64: the wide kernel (128-row
  // blocks, 32 rows per wave). On an MI355X: GPT-2-small attention (T 1024) 0.475 -> 0.412 ms
  // per forward; ViT-S/4 (T 65, one block per image and head instead of a 64-row block and a
  // one-row block that repeats every K/V load) 0.435 -> 0.375 ms
  if (seq_q > 64 && head_dim <= 64) {
    const int64_t nqb = (seq_q + 127) / 128;
    TL_REQUIRE(nqb <= 65535, "too many 128-row query blocks");
    const dim3 grid((unsigned)(batch * n_heads_q), (unsigned)nqb);
    if (causal && nqb > 1) {
      const int per_cu = head_dim == 32 ? wide_blocks_per_cu<32>() : wide_blocks_per_cu<64>();
      const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
      if (per_cu > 0 && (int64_t)grid.x * nqb <= per_cu * cus) p.fold = (int)cus;
    }
    if (head_dim == 32) attention_fwd_wide_kernel<32><<<grid, 256, 0, ctx->stream>>>(p);
    else attention_fwd_wide_kernel<64><<<grid, 256, 0, ctx->stream>>>(p);
    return ls.finish("attention_fwd_wide");
  }
  // head dims 128 and 256 beyond 64 query rows: 8 waves of 16 rows per workgroup (two per
  // SIMD), 128-row blocks
  const int64_t rb = head_dim >= 128 && seq_q > 64 ? 128 : 64;
  const int64_t nqb = (seq_q + rb - 1) / rb;
  dim3 grid((unsigned)(causal ? (nqb + 1) / 2 : nqb), (unsigned)(batch * n_heads_q));
  if (rb == 128) {
    if (head_dim == 128) attention_fwd_kernel<128, 8><<<grid, 512, 0, ctx->stream>>>(p);
    else attention_fwd_kernel<256, 8><<<grid, 512, 0, ctx->stream>>>(p);
    return ls.finish("attention_fwd");
  }
  switch (head_dim) {
    case 32: attention_fwd_kernel<32><<<grid, 256, 0, ctx->stream>>>(p); break;
    case 64: attention_fwd_kernel<64><<<grid, 256, 0, ctx->stream>>>(p); break;
    case 128: attention_fwd_kernel<128><<<grid, 256, 0, ctx->stream>>>(p); break;
    default: attention_fwd_kernel<256><<<grid, 256, 0, ctx->stream>>>(p); break;
  }
  return ls.finish("attention_fwd");
}

extern "C" int tl_attention_fwd(tl_ctx* ctx, const void* q, const void* k, const void* vt,
                                void* out, int64_t batch, int64_t n_heads_q, int64_t n_heads_kv,
                                int64_t seq_q, int64_t seq_k, int64_t head_dim, int64_t ld_out,
                                int64_t offset, float divisor, int32_t causal,
                                int64_t kv_capacity, int32_t dtype) {
  return attention_fwd(ctx, q, k, vt, out, batch, n_heads_q, n_heads_kv, seq_q, seq_k, head_dim,
                       ld_out, offset, divisor, causal, kv_capacity, dtype, false);
}

extern "C" int tl_attention_decode_dev(tl_ctx* ctx, const void* q, void* k,
                                       const void* vt, void* out, int64_t batch,
                                       int64_t n_heads_q, int64_t n_heads_kv, int64_t seq_q,
                                       int64_t head_dim, int64_t ld_out, float divisor,
                                       int64_t kv_capacity, const int64_t* pos,
                                       const void* rope_table, int32_t dtype) {
  if (!pos) {
    (void)enter(ctx);
    return fail(TL_ERR_INVALID, "null position");
  }
  return attention_fwd(ctx, q, k, vt, out, batch, n_heads_q, n_heads_kv, seq_q, kv_capacity,
                       head_dim, ld_out, 0, divisor, 1, kv_capacity, dtype, false, pos,
                       (const float*)rope_table);
}

extern "C" int tl_attention_fwd_noalloc(tl_ctx* ctx, const void* q, const void* k,
                                        const void* vt, void* out, int64_t batch,
                                        int64_t n_heads_q, int64_t n_heads_kv, int64_t seq_q,
                                        int64_t seq_k, int64_t head_dim, int64_t ld_out,
                                        int64_t offset, float divisor, int32_t causal,
                                        int64_t kv_capacity, int32_t dtype) {
  return attention_fwd(ctx, q, k, vt, out, batch, n_heads_q, n_heads_kv, seq_q, seq_k, head_dim,
                       ld_out, offset, divisor, causal, kv_capacity, dtype, true);
}
