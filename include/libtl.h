/*
 * libtl — C ABI of the MI355X (gfx950) runtime behind torchless-nn's Layer interface.
 *
 * The reference library has no native boundary: every `xp.*` expression in a Layer's
 * forward is a CuPy (CUDA) or NumPy (CPU) call, chosen at import by XP_RUNTIME
 * (reference backend.py:3-22). This library is what the new XP_RUNTIME=MI355X value binds
 * through ctypes. Each entry point below names the reference expression(s) it replaces.
 *
 * Conventions
 *  - Every function returns an int status (TL_OK == 0) and never throws. On failure the
 *    message is available from tl_last_error() on the calling thread.
 *  - Device buffers are plain pointers obtained from tl_malloc. The caller owns them; the
 *    library keeps no pointer after a call returns.
 *  - All compute calls are asynchronous enqueues on the context's single in-order HIP
 *    stream. tl_memcpy_d2h, tl_memcpy2d_d2h and tl_sync block. Data errors detected
 *    inside kernels (e.g. an out-of-range token id) are latched in a device status word
 *    and reported, as TL_ERR_BAD_INPUT, by the next blocking call.
 *  - Sizes, leading dimensions and strides are int64 and counted in elements.
 *  - A context must not be used by two host threads at once.
 */
#ifndef LIBTL_H
#define LIBTL_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct tl_ctx tl_ctx;
typedef struct tl_graph tl_graph;

/* Element types. Floating-point data is fp32 or bf16 (bf16 stored as raw uint16). */
enum tl_dtype { TL_F32 = 0, TL_BF16 = 1, TL_I32 = 2, TL_I64 = 3, TL_U8 = 4 };

enum tl_status {
  TL_OK = 0,
  TL_ERR_INVALID = 1,     /* bad argument: null pointer, bad shape, bad enum */
  TL_ERR_HIP = 2,         /* a HIP runtime call failed */
  TL_ERR_OOM = 3,         /* device allocation failed after emptying the cache */
  TL_ERR_NO_DEVICE = 4,   /* no HIP device, or the index is out of range */
  TL_ERR_BAD_INPUT = 5,   /* a kernel saw invalid data (latched, reported at sync) */
  TL_ERR_UNSUPPORTED = 6  /* valid request this build does not implement */
};

/* Activations (reference activations.py). */
enum tl_act { TL_ACT_NONE = 0, TL_ACT_GELU = 1, TL_ACT_SILU = 2 };

/* Layout of the GEMM B operand. */
enum tl_b_layout {
  TL_B_NK = 0, /* B given as Bt[n*ldb + k]  (C = A * Bt^T; weights pre-packed, tied head) */
  TL_B_KN = 1  /* B given as B[k*ldb + n]   (C = A * B, the reference's `x @ W`) */
};

/* Epilogue variants of tl_gemm. */
enum tl_epilogue {
  TL_EPI_STORE = 0,     /* C[m,n] = f(acc) */
  /* scatter [M = B*T, (Hq+2*Hkv)*Dh] into q [B,Hq,T,Dh] and a key/value cache
   * k [B,Hkv,L,Dh], vt [B,Hkv,Dh,L] (L = kv_len, rows written at kv_pos0 + t) */
  TL_EPI_QKV_SPLIT = 1,
  /* GeGLU: B rows interleave gate and up projections (row 2f = gate f, 2f+1 = up f);
   * C[m, f] = gelu(acc[m, 2f]) * acc[m, 2f+1], C is [M, N/2] */
  TL_EPI_GEGLU = 2
};

/* Output tile shapes (rows x columns) of the bf16 MFMA GEMM, for tl_gemm_desc.tile. */
enum tl_gemm_tile {
  TL_TILE_AUTO = 0,
  TL_TILE_256x256 = 1,
  TL_TILE_256x128 = 2,
  TL_TILE_128x128 = 3,
  TL_TILE_128x64 = 4,
  TL_TILE_64x64 = 5,
  TL_TILE_256x256_W4 = 6, /* 256x256 with 4 waves (128x128 per wave); TL_TILE_256x256 uses 8 */
  TL_TILE_256x128_W8 = 7, /* 256x128 with 8 waves (64x64 per wave); TL_TILE_256x128 uses 4 */
  /* direct global->LDS variants (K % 64 == 0; other K fall back to TL_TILE_128x128) */
  TL_TILE_DMA_128x128 = 8,     /* 2 stages */
  TL_TILE_DMA_256x128_W8 = 9,  /* 8 waves, 3 stages */
  TL_TILE_DMA_128x64_S3 = 10,  /* 3 stages */
  TL_TILE_DMA_128x128_S3 = 11, /* 3 stages */
  /* persistent direct-to-LDS variants: one workgroup per resident slot, the next tile's first
   * K steps loaded while the current tile stores its epilogue. bf16 output with plain, bias,
   * bias+activation or residual epilogue, batch 1, N % 8 == 0; other calls run the
   * non-persistent tile of the same shape */
  TL_TILE_PERSIST_256x128_W8 = 12,
  TL_TILE_PERSIST_128x128 = 13,
  /* weight streaming for M <= 16 (decode steps): 16 rows of B per workgroup, K split over
   * its 8 waves; chosen by TL_TILE_AUTO whenever M <= 16 */
  TL_TILE_SKINNY = 14,
  TL_TILE_DMA_256x256_W8 = 15, /* direct global->LDS, 8 waves of 128x64, 2 stages */
  TL_TILE_DMA_128x96 = 16,     /* direct global->LDS, 4 waves of 64x48, 2 stages */
  TL_TILE_DMA_256x96_W8 = 17,  /* direct global->LDS, 8 waves of 64x48, 3 stages */
  TL_TILE_PERSIST_256x96_W8 = 18,  /* persistent (see above), 3 stages */
  TL_TILE_PERSIST_256x256_W8 = 19, /* persistent (see above), 2 stages */
  TL_TILE_DMA_256x192_W8 = 20      /* direct global->LDS, 8 waves of 64x96, 2 stages */
};

/* Kernel families for the built-in per-launch event profiler (tl_kprof_*). */
enum tl_kfamily {
  TL_KF_GEMM_MFMA = 0,  /* bf16 MFMA GEMM, dense projections and LM head */
  TL_KF_GEMM_BATCHED = 1, /* bf16 MFMA GEMM, batched attention products (QK^T, PV) */
  TL_KF_GEMM_SIMT = 2,  /* generic VALU GEMM (fp32 and unaligned shapes) */
  TL_KF_LAYERNORM = 3,
  TL_KF_RMSNORM = 4,
  TL_KF_SOFTMAX = 5,
  TL_KF_ROPE = 6,
  TL_KF_ACT = 7,
  TL_KF_EMBED = 8,
  TL_KF_ARGMAX = 9,
  TL_KF_ATTENTION = 10, /* fused causal attention */
  TL_KF_MISC = 11,      /* fill, cast, transpose, add */
  TL_KF_COUNT = 12
};

/* Argument block of tl_gemm: C = epilogue(A * op(B)), batched over z in [0, batch).
 * z splits as zo = z / batch_inner, zi = z % batch_inner and every operand pointer
 * advances by zo*s?_o + zi*s?_i elements. Epilogue order, per element:
 *   v = acc; if (divisor != 1) v = v / divisor; if (bias) v += bias[n];
 *   v = act(v); if (residual) v += residual[m*ldr + n]; store v in dtype_out. */
typedef struct tl_gemm_desc {
  int64_t M, N, K;
  const void* A; int64_t lda;
  const void* B; int64_t ldb; int32_t b_layout;
  void* C; int64_t ldc;
  int32_t dtype_in, dtype_out;
  int64_t batch, batch_inner;
  int64_t sa_o, sa_i, sb_o, sb_i, sc_o, sc_i;
  const void* bias;                     /* [N], dtype_in, or NULL */
  const void* residual; int64_t ldr;    /* dtype_out, or NULL */
  int64_t sr_o, sr_i;
  int32_t act;                          /* enum tl_act */
  float divisor;
  int32_t epilogue;                     /* enum tl_epilogue */
  void* q; void* k; void* vt;           /* TL_EPI_QKV_SPLIT outputs */
  int64_t seq_len, n_heads_q, n_heads_kv, head_dim;
  int64_t kv_len, kv_pos0;              /* cache capacity (0: seq_len) and write position */
  int32_t family;                       /* enum tl_kfamily used by the profiler */
  int32_t tile;                         /* MFMA tile hint: 0 = choose automatically, else
                                           enum tl_gemm_tile */
  const void* kv_pos0_dev;              /* TL_EPI_QKV_SPLIT: when not NULL, an int64 in device
                                           memory read at run time in place of kv_pos0 (a
                                           captured graph writes the cache at the current
                                           position); rows past kv_len are not written */
  int32_t norm_rows;                    /* nonzero: row m of the product is multiplied by
                                           1 / sqrt(mean_k A[m, k]^2 + norm_eps) before the
                                           epilogue; with an RMSNorm's gain folded into B's
                                           K index that is RMSNorm(A) @ B (unbatched bf16,
                                           M <= 16, B as [N, K] only) */
  float norm_eps;
} tl_gemm_desc;

/* ---- runtime ------------------------------------------------------------------------ */
int tl_version(void);
/* Message of the last failed call on this thread ("" if none). */
const char* tl_last_error(void);
int tl_device_count(int* count);
/* Replaces the CUDA runtime selection at reference backend.py:7-18. */
int tl_init(int device, tl_ctx** out);
int tl_destroy(tl_ctx* ctx);
/* Caching allocator (stream-ordered reuse on the context stream). Replaces CuPy's pool
 * behind every fresh `xp` array a forward allocates (e.g. reference layers.py:208). */
int tl_malloc(tl_ctx* ctx, size_t bytes, void** ptr);
int tl_free(tl_ctx* ctx, void* ptr);
int tl_empty_cache(tl_ctx* ctx);
int tl_mem_stats(tl_ctx* ctx, size_t* bytes_in_use, size_t* bytes_cached);
/* Size of the context's grow-only workspace (the split reductions' partial results), 0 until
 * a call first needs it. No reference counterpart (CuPy's pool has no such buffer). */
int tl_workspace_bytes(tl_ctx* ctx, size_t* bytes);
/* Host<->device copies. Replace `xp.array(host)` (reference network.py:117-118, 152-153) and
 * `.get()` (reference demo.ipynb:1535). h2d returns once the host buffer may be reused: up to
 * 64 MiB it is copied into a pinned staging buffer and the device copy is queued behind the
 * work already on the stream, without waiting for it; larger copies wait for the stream. */
int tl_memcpy_h2d(tl_ctx* ctx, void* dst, const void* src, size_t bytes);
int tl_memcpy_d2h(tl_ctx* ctx, void* dst, const void* src, size_t bytes);
int tl_memcpy_d2d(tl_ctx* ctx, void* dst, const void* src, size_t bytes);
int tl_memcpy2d_h2d(tl_ctx* ctx, void* dst, size_t dpitch, const void* src, size_t spitch,
                    size_t width_bytes, size_t rows);
int tl_memcpy2d_d2h(tl_ctx* ctx, void* dst, size_t dpitch, const void* src, size_t spitch,
                    size_t width_bytes, size_t rows);
/* Device-to-device copy of `rows` rows of width_bytes (stream-ordered): the row copies of
 * `xp.concatenate((tokens, out), axis=1)` (reference demo.ipynb:1533). */
int tl_memcpy2d_d2d(tl_ctx* ctx, void* dst, size_t dpitch, const void* src, size_t spitch,
                    size_t width_bytes, size_t rows);
/* Waits for the stream, then reports any latched kernel data error. */
int tl_sync(tl_ctx* ctx);
/* Cache warming, no reference counterpart (the reference leaves memory traffic to
 * CuPy/NumPy). Names a device region (4-byte aligned, up to 4 regions per launch) that the
 * next tl_layernorm_fwd / tl_rmsnorm_fwd on this context also reads, one word per 128-byte
 * line, so a weight that the product after the norm reads arrives from the device caches
 * instead of HBM. Advisory: results do not change, the values read are discarded, and the
 * list is cleared by that launch. A norm over too few rows to give every CU a workgroup (a
 * decode step) ignores the list (and still clears it). The region must lie inside one live tl_malloc block
 * (TL_ERR_INVALID otherwise); freeing that block drops it from the list. In a captured graph
 * the region is read on every replay, so it must stay allocated while the graph lives. */
int tl_prefetch_hint(tl_ctx* ctx, const void* ptr, int64_t bytes);
/* HIP graphs of the context stream, for replaying a whole step (a decode step, a short
 * forward) with one launch instead of one host call per kernel. No reference counterpart
 * (the reference dispatches every op from Python, network.py:36-39).
 * tl_graph_begin starts capturing: the calls that follow are recorded, not run, until
 * tl_graph_end, which instantiates them. While a capture is open, calls that wait for the
 * stream (tl_sync, host copies) fail with TL_ERR_INVALID, the kernel profiler records
 * nothing, and a workspace that would have to grow fails the call (run the step once
 * before capturing it). Device blocks that tl_malloc hands out during the capture belong to
 * the graph until tl_graph_destroy: replays write them, so they are kept from reuse even
 * after the caller frees them. tl_graph_launch replays the graph on the context stream. */
int tl_graph_begin(tl_ctx* ctx);
int tl_graph_end(tl_ctx* ctx, tl_graph** out);
int tl_graph_launch(tl_ctx* ctx, tl_graph* graph);
int tl_graph_destroy(tl_ctx* ctx, tl_graph* graph);
/* Events on the context stream, for timing. */
int tl_event_create(tl_ctx* ctx, void** ev);
int tl_event_record(tl_ctx* ctx, void* ev);
int tl_event_elapsed_ms(void* start, void* stop, float* ms);
int tl_event_destroy(void* ev);
/* Per-launch event profiler: while enabled for a family mask, every launch of a kernel of
 * those families is bracketed by events; tl_kprof_query sums them after a sync. */
int tl_kprof_enable(tl_ctx* ctx, uint32_t family_mask);
int tl_kprof_reset(tl_ctx* ctx);
int tl_kprof_query(tl_ctx* ctx, int family, int64_t* launches, double* total_ms,
                   double* flops, double* bytes);

/* ---- elementwise helpers -------------------------------------------------------------- */
/* y[i] = value (a kernel, not hipMemset, so it is safe under graph capture).
 * Replaces init_zeros_tensor (reference backend.py:33-34). */
int tl_fill(tl_ctx* ctx, void* y, int64_t n, int32_t dtype, double value);
/* y[i] = x[i] converted (fp32 <-> bf16 with round-to-nearest-even, or a copy). x and y may
 * be the same pointer only when the types match; otherwise they must not overlap. */
int tl_cast(tl_ctx* ctx, const void* x, void* y, int64_t n, int32_t dtype_x, int32_t dtype_y);
/* y[e] = mean + std * N(0,1), drawn on the device: Philox4x32-10 keyed by `seed` with
 * counter (e / 4, stream), Box-Muller on its output word pairs. Replaces
 * init_random_tensor's draw (reference backend.py:27-31, a device draw under CuPy). */
int tl_random_normal(tl_ctx* ctx, void* y, int64_t n, uint64_t seed, uint64_t stream,
                     float mean, float std_dev, int32_t dtype);
/* n draws from the categorical distribution p[0 .. cols) (fp32 or bf16, not necessarily
 * normalised): draw j takes u = (w0 >> 8) 2^-24 from Philox counter (j, 0, stream) under key
 * `seed` and returns the smallest i with p[0] + .. + p[i] > u * sum(p) (the last index if
 * rounding leaves none), as int64. Replaces `xp.random.choice(..., p=probs)` (reference
 * demo.ipynb:1531, CuPy's cumsum + searchsorted). */
int tl_sample(tl_ctx* ctx, const void* probs, int64_t cols, int32_t dtype, int64_t n,
              uint64_t seed, uint64_t stream, int64_t* out);
/* out[i] = src[idx[i]] for elements of elem_bytes (1, 2, 4, 8) bytes; an index outside
 * [0, src_len) is reported as TL_ERR_BAD_INPUT at the next synchronising call. The gather
 * of `xp.random.choice(a, ...)` from its candidate array `a`. */
int tl_take(tl_ctx* ctx, const void* src, int64_t src_len, int32_t elem_bytes,
            const int64_t* idx, int64_t n, void* out);
/* y[c*ldy + r] = x[r*ldx + c]: weight pre-packing into the K-contiguous GEMM layout. */
int tl_transpose2d(tl_ctx* ctx, const void* x, void* y, int64_t rows, int64_t cols,
                   int64_t ldx, int64_t ldy, int32_t dtype);
/* y[c, r] = x[r, c] * (gain_offset + gain[r]) (float types; gain has `rows` elements): the
 * transpose that packs a [K, N] weight as [N, K] with an RMSNorm's gain folded into K, for
 * products that take the norm as row scaling (tl_gemm_desc.norm_rows). */
int tl_transpose2d_gain(tl_ctx* ctx, const void* x, void* y, int64_t rows, int64_t cols,
                        int64_t ldx, int64_t ldy, const void* gain, float gain_offset,
                        int32_t dtype);
/* ViT patch extraction, reference transformer_adapters.py:39-47 (VitProjector.forward's
 * reshape / transpose(0,2,4,3,5,1) / reshape): x [B, C, H, W] -> y [B, (H/ph)(W/pw),
 * ph*pw*C], token i*(W/pw) + j, features ordered (row in patch, column in patch, channel).
 * H and W must be multiples of the patch size. x and y may differ in dtype. */
int tl_patchify(tl_ctx* ctx, const void* x, void* y, int64_t batch, int64_t channels,
                int64_t height, int64_t width, int64_t patch_h, int64_t patch_w,
                int32_t dtype_x, int32_t dtype_y);
/* The whole ViT front end in one launch, reference transformer_adapters.py:34-55
 * (VitProjector.forward: patches, @ projection, class/register tokens prepended, + positions):
 * out [B, R + L, dim] with rows r < R = n_cls_reg equal to cls_reg[r] + pos[r] and rows
 * R + l equal to patches(x)[b, l] @ w^T + pos[R + l] for the L = (H/ph)(W/pw) patches
 * (features in (row in patch, column in patch, channel) order, as tl_patchify). w is the
 * projection given as [dim, K], K = ph pw C. bf16 only, K <= 64 and a multiple of 8, L <= 64,
 * dim a multiple of 96 and at most 4096, n_cls_reg <= 64, C H W <= 2^24, w and out 16-byte
 * aligned, cls_reg and pos 8-byte aligned; other shapes return TL_ERR_UNSUPPORTED
 * (tl_patchify, tl_gemm and tl_embed_fwd compose the same result). Equal bit for bit to
 * that composition. */
int tl_vit_project(tl_ctx* ctx, const void* x, const void* w, const void* cls_reg,
                   const void* pos, void* out, int64_t batch, int64_t channels, int64_t height,
                   int64_t width, int64_t patch_h, int64_t patch_w, int64_t dim,
                   int64_t n_cls_reg, int32_t dtype);
/* y = a + b (elementwise, same shape). Replaces the residual adds at reference
 * layers.py:465-466 when they are not fused into a GEMM epilogue. */
int tl_add(tl_ctx* ctx, const void* a, const void* b, void* y, int64_t n, int32_t dtype);

/* ---- the hot path --------------------------------------------------------------------- */
/* out[i, :] = table[ids[i], :] * scale + pos[pos0 + i % seq_len, :]  (pos may be NULL).
 * Replaces GPTEmbedFront.forward (reference transformer_adapters.py:148-153; scale 1 there).
 * Ids outside [0, vocab) zero the row and latch TL_ERR_BAD_INPUT. */
int tl_embed_fwd(tl_ctx* ctx, const void* ids, int32_t ids_dtype, const void* table,
                 const void* pos, void* out, int64_t n_tokens, int64_t seq_len, int64_t pos0,
                 int64_t vocab, int64_t dim, int64_t ld_out, float scale, int32_t dtype);
/* y = (x - mean) / sqrt(var + eps) * gamma + beta per row (population variance).
 * Replaces LayerNorm.forward (reference layers.py:415-428). */
int tl_layernorm_fwd(tl_ctx* ctx, const void* x, const void* gamma, const void* beta, void* y,
                     int64_t rows, int64_t cols, int64_t ldx, int64_t ldy, float eps,
                     int32_t dtype);
/* y = x / sqrt(mean(x^2) + eps) * (gamma_offset + gamma) per row. No reference counterpart
 * (the reference has only a TODO for it, layers.py:394). */
int tl_rmsnorm_fwd(tl_ctx* ctx, const void* x, const void* gamma, void* y, int64_t rows,
                   int64_t cols, int64_t ldx, int64_t ldy, float eps, float gamma_offset,
                   int32_t dtype);
/* y = exp((x - max)/temperature) / sum(...) per row. With causal != 0, row r only attends
 * to columns j <= (r % period) + offset; the others get exactly 0. Replaces the attention
 * softmax with its -1e9 additive mask (reference layers.py:295-300) and SoftMax.forward
 * (reference activations.py:57-64). */
int tl_softmax_fwd(tl_ctx* ctx, const void* x, void* y, int64_t rows, int64_t cols,
                   int64_t ldx, int64_t ldy, float temperature, int32_t causal, int64_t period,
                   int64_t offset, int32_t dtype);
/* table (fp32, [2][T][D/2]: cos block then sin block) of angles (pos0 + t) * base^(-2i/D),
 * evaluated in fp64. No reference counterpart (positions are absolute there). */
int tl_rope_table(tl_ctx* ctx, void* table, int64_t seq_len, int64_t head_dim, double base,
                  int64_t pos0);
/* tl_rope_table for positions *pos0 .. *pos0 + seq_len - 1, with *pos0 an int64 read from
 * device memory when the kernel runs (a graph replays it at the current position). */
int tl_rope_table_dev(tl_ctx* ctx, void* table, int64_t seq_len, int64_t head_dim, double base,
                      const int64_t* pos0);
/* In-place tl_rope2_fwd whose second set starts at row *pos of each sequence: x2 points at
 * row 0 of n_seq2 sequences of rows_cap2 rows, seq_stride2 elements apart (a KV cache), and
 * rows *pos .. *pos + seq_len - 1 of each are rotated by the table's seq_len positions
 * (rows at or past rows_cap2 are skipped). *pos is an int64 read from device memory when
 * the kernel runs. */
int tl_rope2_dev(tl_ctx* ctx, void* x1, int64_t n_seq1, int64_t seq_stride1, void* x2,
                 int64_t n_seq2, int64_t seq_stride2, int64_t rows_cap2, const void* table,
                 int64_t seq_len, int64_t head_dim, const int64_t* pos, int32_t dtype);
/* *x += delta on the device (advances a device position inside a graph). */
int tl_i64_add(tl_ctx* ctx, int64_t* x, int64_t delta);
/* hist[r * ld_hist + (*pos - pos_base)] = ids[r] for r < rows, when that column lies in
 * [0, cols): records a decode step's token ids at a device position. */
int tl_ids_append(tl_ctx* ctx, const int64_t* ids, int64_t* hist, int64_t rows, int64_t ld_hist,
                  int64_t cols, const int64_t* pos, int64_t pos_base);
/* Rotate-half RoPE over x [n_seq][seq_stride] holding T rows of D (row pitch D) per
 * sequence (seq_stride = T*D when packed; a cache slice uses its capacity * D): for i < D/2,
 * y[i] = x[i] cos - x[i+D/2] sin, y[i+D/2] = x[i+D/2] cos + x[i] sin. In place is allowed. */
int tl_rope_fwd(tl_ctx* ctx, const void* x, void* y, const void* table, int64_t n_seq,
                int64_t seq_len, int64_t head_dim, int64_t seq_stride, int32_t dtype);
/* tl_rope_fwd over two tensors rotated by the same T positions, in one launch: set 1 is
 * (x1, y1, n_seq1, seq_stride1), set 2 (x2, y2, n_seq2, seq_stride2); either set may be
 * empty (n_seq 0, pointers may then be null). Used for the queries and the new cache keys
 * of one multi-query attention call. No reference counterpart (the reference has no RoPE). */
int tl_rope2_fwd(tl_ctx* ctx, const void* x1, void* y1, int64_t n_seq1, int64_t seq_stride1,
                 const void* x2, void* y2, int64_t n_seq2, int64_t seq_stride2,
                 const void* table, int64_t seq_len, int64_t head_dim, int32_t dtype);
/* Replaces GeLU.forward / SiLU.forward (reference activations.py:24-28, 41-45). */
int tl_act_fwd(tl_ctx* ctx, const void* x, void* y, int64_t n, int32_t act, int32_t dtype);
/* out[r] = first index of the maximum of row r (NaN counts as the maximum), int64.
 * Replaces xp.argmax(y_hat, axis=-1) (reference network.py:135, 158). */
int tl_argmax(tl_ctx* ctx, const void* x, int64_t rows, int64_t cols, int64_t ldx,
              int32_t dtype, void* out_ids);
/* Every matmul of the forward: reference layers.py:208, 286, 293, 303, 306, 372, 373,
 * transformer_adapters.py:49, 93, 176. */
int tl_gemm(tl_ctx* ctx, const tl_gemm_desc* desc);
/* Fused causal attention for q [B, Hq, Tq, D], k [B, Hkv, Lk, D], vt [B, Hkv, D, Lk] of which
 * the first seq_k keys are valid (Lk = kv_capacity, 0 meaning seq_k; positions at or past
 * seq_k may hold anything, NaN included: they are never read as scores or values, because
 * the kernels zero what they load from there): out[b, t, h*D + d] with row pitch ld_out, scores
 * divided by `divisor`; query head h reads kv head h / (Hq / Hkv); query t sits at key
 * position t + offset. Replaces reference layers.py:293-304 (scores, mask, softmax, P.V,
 * head merge) in one kernel. */
int tl_attention_fwd(tl_ctx* ctx, const void* q, const void* k, const void* vt, void* out,
                     int64_t batch, int64_t n_heads_q, int64_t n_heads_kv, int64_t seq_q,
                     int64_t seq_k, int64_t head_dim, int64_t ld_out, int64_t offset,
                     float divisor, int32_t causal, int64_t kv_capacity, int32_t dtype);
/* Causal decode attention (at most 16 query rows per kv head) at a device position: query t
 * sits at position *pos + t and keys 0 .. *pos + seq_q - 1 of the cache (capacity
 * kv_capacity, at most that many) are attended to, with *pos an int64 read from device
 * memory when the kernels run, so a captured decode step replays at the current position.
 * Otherwise as tl_attention_fwd. With rope_table (float [2, seq_q, head_dim/2]: cos then
 * sin of positions *pos ..; head_dim >= 64), q and the cache keys at positions *pos ..
 * *pos + seq_q - 1 are taken unrotated: the kernel applies rotate-half RoPE to both and
 * writes the rotated keys back into k. No reference counterpart (the reference recomputes
 * the window every step, demo.ipynb:1526-1533). */
int tl_attention_decode_dev(tl_ctx* ctx, const void* q, void* k, const void* vt, void* out,
                            int64_t batch, int64_t n_heads_q, int64_t n_heads_kv, int64_t seq_q,
                            int64_t head_dim, int64_t ld_out, float divisor, int64_t kv_capacity,
                            const int64_t* pos, const void* rope_table, int32_t dtype);
/* tl_attention_fwd that allocates nothing: the same arguments, kernels and results, with the
 * decode path's partial results (at most 16 query rows per kv head) kept in a static device
 * array of 16 MiB instead of the context's grow-only workspace, and the launch kept out of the
 * event profiler. No counterpart in the reference; it is for callers that cannot allocate
 * (code under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc). A
 * call whose partials need more than 16 MiB (batch x kv heads x key blocks of 64 keys, each
 * 16 x (head_dim + 2) floats) fails with TL_ERR_INVALID. Every call on one GPU shares that
 * GPU's array, which keeps the last call's contents. Eager calls from different contexts take
 * it in turn: a call first makes its context's stream wait (on the device, with no host wait)
 * for the event recorded after the last call from another context. A call made while the
 * stream is being captured into a graph is outside that order: replaying the graph while
 * another context's call is in flight on the same GPU races with it. */
int tl_attention_fwd_noalloc(tl_ctx* ctx, const void* q, const void* k, const void* vt,
                             void* out, int64_t batch, int64_t n_heads_q, int64_t n_heads_kv,
                             int64_t seq_q, int64_t seq_k, int64_t head_dim, int64_t ld_out,
                             int64_t offset, float divisor, int32_t causal,
                             int64_t kv_capacity, int32_t dtype);

#ifdef __cplusplus
}
#endif
#endif /* LIBTL_H */
