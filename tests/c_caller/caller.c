/*
 * A C caller of libmoe_hip built against include/moe_hip.h alone, calling
 * the drop-in entry points the way the reference's own code would after the
 * integration patches: block_forward's moe_forward (src/transformer.c:761-764)
 * and its whole FFN half (moe_block_ffn, :760-767), and inference_step's MoE
 * slot (moe_decode_step, src/inference.c:342-343).
 *
 * Usage: caller DIR.  DIR holds raw little-endian files written by the test:
 *   shape.i32  T d F E k
 *   x.f32 [T x d], wr.f32 [d x E], wg.f32 / wu.f32 [E][d x F], wd.f32 [E][F x d],
 *   rms.f32 [d], xd.f32 [d] (decode residual row), xnd.f32 [d] (its x_norm)
 * and receives
 *   out.f32, probs.f32, ids.i32 (moe_forward), blk_x.f32, blk_xn.f32, blk_fo.f32,
 *   blk_probs.f32, blk_ids.i32 (moe_block_ffn on a copy of x), dec_x.f32
 *   (moe_decode_step).
 * Exit status 0 on success.
 */
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "moe_hip.h"

static char g_dir[4096];

static void *load(const char *name, size_t bytes) {
    char path[4200];
    snprintf(path, sizeof(path), "%s/%s", g_dir, name);
    FILE *f = fopen(path, "rb");
    if (!f) { fprintf(stderr, "cannot open %s\n", path); exit(2); }
    void *p = malloc(bytes ? bytes : 1);
    if (!p || fread(p, 1, bytes, f) != bytes) { fprintf(stderr, "short read %s\n", path); exit(2); }
    fclose(f);
    return p;
}

static void save(const char *name, const void *p, size_t bytes) {
    char path[4200];
    snprintf(path, sizeof(path), "%s/%s", g_dir, name);
    FILE *f = fopen(path, "wb");
    if (!f || fwrite(p, 1, bytes, f) != bytes) { fprintf(stderr, "cannot write %s\n", path); exit(2); }
    fclose(f);
}

static Matrix view(float *data, int rows, int cols) {
    Matrix m;
    m.data = data;
    m.grad = NULL;
    m.rows = rows;
    m.cols = cols;
    return m;
}

int main(int argc, char **argv) {
    if (argc != 2) { fprintf(stderr, "usage: %s DIR\n", argv[0]); return 2; }
    snprintf(g_dir, sizeof(g_dir), "%s", argv[1]);
    int *sh = (int *)load("shape.i32", 5 * sizeof(int));
    const int T = sh[0], d = sh[1], F = sh[2], E = sh[3], k = sh[4];
    const size_t dF = (size_t)d * F;
    float *x = (float *)load("x.f32", sizeof(float) * (size_t)T * d);
    float *wr = (float *)load("wr.f32", sizeof(float) * (size_t)d * E);
    float *wg = (float *)load("wg.f32", sizeof(float) * E * dF);
    float *wu = (float *)load("wu.f32", sizeof(float) * E * dF);
    float *wd = (float *)load("wd.f32", sizeof(float) * E * dF);
    float *rms = (float *)load("rms.f32", sizeof(float) * (size_t)d);
    float *xd = (float *)load("xd.f32", sizeof(float) * (size_t)d);
    float *xnd = (float *)load("xnd.f32", sizeof(float) * (size_t)d);

    /* The model's structs as the reference lays them out (include/transformer.h). */
    FFNWeights *ex = (FFNWeights *)calloc((size_t)E, sizeof(FFNWeights));
    for (int e = 0; e < E; ++e) {
        ex[e].W_gate = view(wg + e * dF, d, F);
        ex[e].W_up = view(wu + e * dF, d, F);
        ex[e].W_down = view(wd + e * dF, F, d);
    }
    MoEWeights mw;
    mw.experts = ex;
    mw.W_router = view(wr, d, E);
    mw.n_experts = E;
    mw.top_k = k;
    ModelConfig cfg;
    memset(&cfg, 0, sizeof(cfg));
    cfg.max_seq_len = T;
    cfg.d_model = d;
    cfg.n_layers = 1;
    cfg.n_heads = 1;
    cfg.n_kv_heads = 1;
    cfg.head_dim = d;
    cfg.ffn_hidden = F;
    cfg.n_experts = E;
    cfg.top_k_experts = k;
    cfg.rms_norm_eps = 1e-5f;
    cfg.rope_theta = 10000.0f;

    /* block_forward's call: moe_forward(&cache->x_norm_ffn, &bw->moe, cfg,
     * cache, &cache->ffn_out), with the cache's routing arrays. */
    float *out = (float *)calloc((size_t)T * d, sizeof(float));
    float *probs = (float *)calloc((size_t)T * E, sizeof(float));
    int *ids = (int *)calloc((size_t)T * k, sizeof(int));
    ForwardCache cache;
    memset(&cache, 0, sizeof(cache));
    cache.router_probs = probs;
    cache.expert_ids = ids;
    Matrix xm = view(x, T, d), om = view(out, T, d);
    moe_forward(&xm, &mw, &cfg, &cache, &om);
    save("out.f32", out, sizeof(float) * (size_t)T * d);
    save("probs.f32", probs, sizeof(float) * (size_t)T * E);
    save("ids.i32", ids, sizeof(int) * (size_t)T * k);

    /* The FFN half of block_forward for a MoE block, on a copy of x. */
    float *bx = (float *)malloc(sizeof(float) * (size_t)T * d);
    memcpy(bx, x, sizeof(float) * (size_t)T * d);
    float *bxn = (float *)calloc((size_t)T * d, sizeof(float));
    float *bfo = (float *)calloc((size_t)T * d, sizeof(float));
    ForwardCache bc;
    memset(&bc, 0, sizeof(bc));
    bc.x_norm_ffn = view(bxn, T, d);
    bc.ffn_out = view(bfo, T, d);
    bc.router_probs = (float *)calloc((size_t)T * E, sizeof(float));
    bc.expert_ids = (int *)calloc((size_t)T * k, sizeof(int));
    Matrix bxm = view(bx, T, d);
    moe_block_ffn(&bxm, rms, &mw, &cfg, &bc);
    save("blk_x.f32", bx, sizeof(float) * (size_t)T * d);
    save("blk_xn.f32", bxn, sizeof(float) * (size_t)T * d);
    save("blk_fo.f32", bfo, sizeof(float) * (size_t)T * d);
    save("blk_probs.f32", bc.router_probs, sizeof(float) * (size_t)T * E);
    save("blk_ids.i32", bc.expert_ids, sizeof(int) * (size_t)T * k);

    /* inference_step's MoE slot: s->x += MoE(s->x_norm) for one sequence. */
    moe_decode_step(&mw, &cfg, xnd, xd);
    save("dec_x.f32", xd, sizeof(float) * (size_t)d);

    if (moe_hip_last_error() != MOE_HIP_OK) {
        fprintf(stderr, "libmoe_hip: %s\n", moe_hip_last_error_message());
        return 1;
    }
    moe_hip_shutdown();
    puts("caller ok");
    return 0;
}
