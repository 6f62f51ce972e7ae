/* ref_ckpt_harness.c — test infrastructure, never shipped or measured.
 *
 * Writes a checkpoint with the reference's own model_save
 * (src/transformer.c:573-616): the caller's arrays are placed in the
 * reference's Model struct field by field (embedding, each block's norm
 * scales and attention matrices, and, for a MoE block, the router and every
 * expert's gate, up and down matrices, then the final norm and the head), and
 * model_save decides what goes where in the file.  Compiled with the
 * reference's sources where they lie (oracle/Makefile, target ref); used by
 * tests/golden/make_moe_ckpt.py only.
 *
 * Arrays per block l are given as arrays of pointers: rms_attn[l], wq[l],
 * wk[l], wv[l], wo[l], rms_ffn[l], wr[l] and, per expert e of block l,
 * wg[l * E + e], wu[...], wd[...].
 */
#include <stdlib.h>
#include <string.h>

#include "transformer.h"

static Matrix view(const float *p, int rows, int cols) {
    Matrix m;
    m.data = (float *)p;
    m.grad = NULL;
    m.rows = rows;
    m.cols = cols;
    return m;
}

int ref_ckpt_save(const char *path, const ModelConfig *cfg, const float *embed,
                  const float *const *rms_attn, const float *const *wq, const float *const *wk,
                  const float *const *wv, const float *const *wo, const float *const *rms_ffn,
                  const float *const *wr, const float *const *wg, const float *const *wu,
                  const float *const *wd, const float *rms_final, const float *lm_head) {
    const int d = cfg->d_model, L = cfg->n_layers, E = cfg->n_experts, F = cfg->ffn_hidden;
    const int qd = cfg->n_heads * cfg->head_dim, kd = cfg->n_kv_heads * cfg->head_dim;
    Model m;
    memset(&m, 0, sizeof m);
    m.cfg = *cfg;
    m.weights.embed = view(embed, cfg->vocab_size, d);
    m.weights.n_layers = L;
    m.weights.blocks = (BlockWeights *)calloc((size_t)L, sizeof(BlockWeights));
    FFNWeights *ex = (FFNWeights *)calloc((size_t)L * (E > 1 ? E : 1), sizeof(FFNWeights));
    if (!m.weights.blocks || !ex) return -2;
    for (int l = 0; l < L; ++l) {
        BlockWeights *b = &m.weights.blocks[l];
        b->rms_attn = (float *)rms_attn[l];
        b->attn.W_Q = view(wq[l], d, qd);
        b->attn.W_K = view(wk[l], d, kd);
        b->attn.W_V = view(wv[l], d, kd);
        b->attn.W_O = view(wo[l], qd, d);
        b->rms_ffn = (float *)rms_ffn[l];
        b->use_moe = E > 1;
        if (b->use_moe) {
            for (int e = 0; e < E; ++e) {
                ex[l * E + e].W_gate = view(wg[l * E + e], d, F);
                ex[l * E + e].W_up = view(wu[l * E + e], d, F);
                ex[l * E + e].W_down = view(wd[l * E + e], F, d);
            }
            b->moe.experts = ex + (size_t)l * E;
            b->moe.W_router = view(wr[l], d, E);
            b->moe.n_experts = E;
            b->moe.top_k = cfg->top_k_experts;
        } else {
            b->ffn.W_gate = view(wg[l], d, F);
            b->ffn.W_up = view(wu[l], d, F);
            b->ffn.W_down = view(wd[l], F, d);
        }
    }
    m.weights.rms_final = (float *)rms_final;
    m.weights.lm_head = view(lm_head, d, cfg->vocab_size);
    const int rc = model_save(&m, path);
    free(m.weights.blocks);
    free(ex);
    return rc;
}
