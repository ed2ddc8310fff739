// Fused causal attention (scores, mask, softmax, P.V and head merge in one kernel).
#include "tl_internal.hpp"

using namespace tl;

extern "C" int tl_attention_fwd(tl_ctx* ctx, const void* q, const void* k, const void* vt,
                                void* out, int64_t batch, int64_t n_heads_q, int64_t n_heads_kv,
                                int64_t seq_q, int64_t seq_k, int64_t head_dim, int64_t ld_out,
                                int64_t offset, float divisor, int32_t causal, int32_t dtype) {
  int rc = enter(ctx);
  if (rc) return rc;
  (void)q; (void)k; (void)vt; (void)out; (void)batch; (void)n_heads_q; (void)n_heads_kv;
  (void)seq_q; (void)seq_k; (void)head_dim; (void)ld_out; (void)offset; (void)divisor;
  (void)causal; (void)dtype;
  return fail(TL_ERR_UNSUPPORTED, "tl_attention_fwd is not implemented yet");
}
