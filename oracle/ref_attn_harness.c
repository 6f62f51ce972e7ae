/* ref_attn_harness.c — test infrastructure, never shipped or measured.
 *
 * Drives the reference's own decode step, inference_step
 * (src/inference.c:231-363), for one token of a one-block model built from
 * the caller's arrays.  The block is a MoE block, whose FFN half the
 * reference's decode path leaves as the identity (src/inference.c:340-342),
 * so after the call x = x + Attn(rmsnorm_vec(x)) exactly as the reference
 * computes it: rmsnorm_vec, the matvec chains, rope_apply_pos, the cache
 * append at `pos`, vec_dot, softmax_vec, vec_axpy, W_O and the residual add
 * (:252-308).  Compiled with the reference's sources where they lie
 * (oracle/Makefile, target ref); used by tests/golden/make_golden.py only.
 */
#include <stdlib.h>
#include <string.h>

#include "inference.h"

int ref_attn_step(int d, int nh, int nkv, int hd, int max_seq, float eps, const float *wq,
                  const float *wk, const float *wv, const float *wo, const float *rms_attn,
                  const float *cos_t, const float *sin_t, float *kc, float *vc, int pos,
                  float *x) {
    if (pos < 0 || pos >= max_seq) return -1;
    const int qd = nh * hd, kd = nkv * hd;
    Model m;
    memset(&m, 0, sizeof m);
    m.cfg.vocab_size = 1;
    m.cfg.max_seq_len = max_seq;
    m.cfg.d_model = d;
    m.cfg.n_layers = 1;
    m.cfg.n_heads = nh;
    m.cfg.n_kv_heads = nkv;
    m.cfg.head_dim = hd;
    m.cfg.n_experts = 2;
    m.cfg.top_k_experts = 1;
    m.cfg.rms_norm_eps = eps;
    m.cfg.rope_theta = 10000.0f;

    float *ones = (float *)malloc(sizeof(float) * d);
    float *head = (float *)calloc((size_t)d, sizeof(float));
    float *row = (float *)malloc(sizeof(float) * d);
    if (!ones || !head || !row) return -2;
    for (int i = 0; i < d; ++i) ones[i] = 1.0f;
    memcpy(row, x, sizeof(float) * d);

    BlockWeights blk;
    memset(&blk, 0, sizeof blk);
    blk.rms_attn = (float *)rms_attn;
    blk.rms_ffn = ones;
    blk.use_moe = 1;
    blk.attn.W_Q = (Matrix){(float *)wq, NULL, d, qd};
    blk.attn.W_K = (Matrix){(float *)wk, NULL, d, kd};
    blk.attn.W_V = (Matrix){(float *)wv, NULL, d, kd};
    blk.attn.W_O = (Matrix){(float *)wo, NULL, qd, d};

    m.weights.embed = (Matrix){row, NULL, 1, d};   /* token 0 -> x */
    m.weights.blocks = &blk;
    m.weights.n_layers = 1;
    m.weights.rms_final = ones;
    m.weights.lm_head = (Matrix){head, NULL, d, 1};
    m.rope = (RoPEBuffer){(float *)cos_t, (float *)sin_t, max_seq, hd};

    InferenceState *s = inference_init(&m);
    const size_t cache = (size_t)max_seq * kd;
    memcpy(s->kv_cache[0].K, kc, sizeof(float) * cache);
    memcpy(s->kv_cache[0].V, vc, sizeof(float) * cache);
    s->seq_pos = pos;
    inference_step(&m, s, 0);
    memcpy(x, s->x, sizeof(float) * d);
    memcpy(kc, s->kv_cache[0].K, sizeof(float) * cache);
    memcpy(vc, s->kv_cache[0].V, sizeof(float) * cache);
    inference_free(s);
    free(ones);
    free(head);
    free(row);
    return 0;
}
