/*
 * moe_hip.h — C ABI of libmoe_hip, the MI355X (gfx950) mixture-of-experts
 * layer that drops into murderface-cpu/llm.c.
 *
 * Reference interfaces this library replaces or extends (paths relative to
 * the reference repo root):
 *   moe_forward        include/transformer.h:270-272, src/transformer.c:287-366
 *                      (caller: block_forward, src/transformer.c:761-764)
 *   moe_decode_step    the empty MoE branch of inference_step,
 *                      src/inference.c:342-343 (x += MoE(x_norm), one row)
 *   moe_decode_batch   the same for n rows at once (the reference decodes one
 *                      sequence per inference_step call, src/inference.c:231)
 * Struct layouts are byte-compatible with include/matrix.h:33-38,
 * include/transformer.h:35-58,108-124 and include/config.h:23-48.  If the
 * reference headers are included first, their definitions are used.
 *
 * Threading: one process-wide HIP stream; calls are serialised by the caller
 * (the reference calls moe_forward from one thread, src/train.c:467-476).
 */
#ifndef MOE_HIP_H
#define MOE_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if !defined(LLM_MATRIX_H)
/* include/matrix.h:33-38 */
typedef struct {
    float *data;
    float *grad;
    int    rows;
    int    cols;
} Matrix;
#endif

#if !defined(LLM_CONFIG_H)
/* include/config.h:23-48 */
typedef struct {
    int vocab_size;
    int max_seq_len;
    int d_model;
    int n_layers;
    int n_heads;
    int n_kv_heads;
    int head_dim;
    int window_size;
    int ffn_hidden;
    int n_experts;
    int top_k_experts;
    float rms_norm_eps;
    float rope_theta;
} ModelConfig;
#endif

#if !defined(LLM_TRANSFORMER_H)
/* include/transformer.h:35-39 */
typedef struct {
    Matrix W_gate;   /* [d_model x ffn_hidden] */
    Matrix W_up;     /* [d_model x ffn_hidden] */
    Matrix W_down;   /* [ffn_hidden x d_model] */
} FFNWeights;

/* include/transformer.h:53-58 */
typedef struct {
    FFNWeights *experts;   /* [n_experts] */
    Matrix      W_router;  /* [d_model x n_experts] */
    int         n_experts;
    int         top_k;
} MoEWeights;

/* include/transformer.h:108-124 */
typedef struct {
    Matrix x_norm_attn, x_norm_ffn, attn_out, ffn_out;
    Matrix Q, K, V;
    Matrix attn_scores, attn_weighted;
    Matrix gate_buf, up_buf;
    float *router_probs;   /* [seq_len x n_experts] */
    int   *expert_ids;     /* [seq_len x top_k]     */
} ForwardCache;
#endif

/* ---------------------------------------------------------------------------
 * Status codes (moe_hip_last_error / status-returning entry points)
 * ------------------------------------------------------------------------- */
enum {
    MOE_HIP_OK = 0,
    MOE_HIP_ERR_ARG = 1,          /* bad shape / null pointer / top_k > n_experts */
    MOE_HIP_ERR_UNSUPPORTED = 2,  /* shape outside the kernels' constraints       */
    MOE_HIP_ERR_HIP = 3,          /* a HIP runtime call failed                    */
    MOE_HIP_ERR_NOMEM = 4,        /* device allocation failed                     */
    MOE_HIP_ERR_NODEV = 5         /* no usable GPU                                */
};

/* ---------------------------------------------------------------------------
 * Drop-in entry points (host pointers, synchronous at return)
 * ------------------------------------------------------------------------- */

/* Replaces moe_forward (include/transformer.h:270-272).  Overwrites out
 * [x->rows x d_model], writes cache->router_probs [T x E] and
 * cache->expert_ids [T x top_k].  Weights are uploaded on first use and kept
 * resident, keyed by the MoEWeights address and every matrix data pointer;
 * call moe_hip_invalidate() after changing weight values in place.  Any
 * d_model and ffn_hidden: widths the kernels do not tile are padded with
 * zeros inside the resident layer (same routing bits, same outputs within
 * the layer tolerance); n_experts <= 4096 and top_k <= 256 (layers past 256
 * experts or top-16 route through general kernels, with the same bits).  The
 * same holds for moe_decode_step, moe_decode_batch and moe_block_ffn.
 * On error it prints the reason and aborts, as the reference does on OOM
 * (src/matrix.c:148-158). */
void moe_forward(const Matrix *x, const MoEWeights *w, const ModelConfig *cfg,
                 ForwardCache *cache, Matrix *out);

/* moe_forward with a status code instead of abort. */
int moe_hip_forward(const Matrix *x, const MoEWeights *w, const ModelConfig *cfg,
                    ForwardCache *cache, Matrix *out);

/* Fills the MoE slot of inference_step (src/inference.c:342-343) for one row:
 * x[0:d] += MoE(x_norm[0:d]).  Aborts on error. */
void moe_decode_step(const MoEWeights *w, const ModelConfig *cfg,
                     const float *x_norm, float *x);

/* Batched decode extension: x[r] += MoE(x_norm[r]) for r < n_rows (one new
 * token for each of n_rows sequences).  Returns a status code. */
int moe_decode_batch(const MoEWeights *w, const ModelConfig *cfg,
                     const float *x_norm, int n_rows, float *x);

/* The FFN half of block_forward for a MoE block (src/transformer.c:760-767):
 * cache->x_norm_ffn = rms_norm(x; rms_ffn, cfg->rms_norm_eps) (src/matrix.c:
 * 666-711), cache->ffn_out = moe_forward(x_norm_ffn) with router_probs and
 * expert_ids, then x += ffn_out.  The normalisation runs on the GPU with the
 * layer; cache->x_norm_ffn and ffn_out must be T x d views.  Aborts on error.
 * The reference build evaluates 1/sqrt with the x86 RSQRTSS estimate and a
 * Newton step; here it is correctly rounded, so x_norm_ffn agrees with the
 * reference's to a few ulp (every later step is the reference's recipe). */
void moe_block_ffn(Matrix *x, const float *rms_ffn, const MoEWeights *w, const ModelConfig *cfg,
                   ForwardCache *cache);
int moe_hip_block_ffn(Matrix *x, const float *rms_ffn, const MoEWeights *w,
                      const ModelConfig *cfg, ForwardCache *cache);

/* ---------------------------------------------------------------------------
 * Library state and residency
 * ------------------------------------------------------------------------- */
int  moe_hip_init(int device);          /* optional; first call does it      */
void moe_hip_shutdown(void);            /* frees every resident buffer       */
int  moe_hip_invalidate(const MoEWeights *w);  /* drop w's device copy       */
int  moe_hip_last_error(void);
const char *moe_hip_error_string(int code);
const char *moe_hip_last_error_message(void);

/* ---------------------------------------------------------------------------
 * Device-resident API: weights packed on the GPU, activations in device
 * memory, work queued on `stream` (a hipStream_t; NULL = the library stream)
 * and NOT synchronised.  Used by callers whose residual stream already lives
 * on the GPU, by the benchmark and by the parity tests.
 * ------------------------------------------------------------------------- */
typedef struct MoeHipLayer MoeHipLayer;

int moe_hip_layer_create(int d_model, int ffn_hidden, int n_experts, int top_k,
                         MoeHipLayer **layer);
int moe_hip_layer_destroy(MoeHipLayer *layer);

/* Upload host weights (reference layout) and pack them. */
int moe_hip_layer_load(MoeHipLayer *layer, const MoEWeights *w);

/* Router bias b[E] added to the logits after the product, as mat_mul_add
 * (src/matrix.c:418-439) does; NULL clears it.  The reference MoE has no
 * router bias (src/transformer.c:299-300): zero bias = reference semantics. */
int moe_hip_layer_set_router_bias(MoeHipLayer *layer, const float *bias);

/* Deterministic synthetic weights generated on the device: W_router ~
 * N(0, std_router), experts ~ N(0, std_expert), streams: router 1, expert e
 * gate 16+3e, up 17+3e, down 18+3e (flat row-major index in each). */
int moe_hip_layer_fill_synthetic(MoeHipLayer *layer, uint64_t seed,
                                 float std_router, float std_expert);

/* Copy expert e back to host in the reference layout (any pointer may be
 * NULL): wg, wu [d x F], wd [F x d]; wr [d x E] via moe_hip_layer_get_router. */
int moe_hip_layer_get_expert(MoeHipLayer *layer, int e, float *wg, float *wu,
                             float *wd);
int moe_hip_layer_get_router(MoeHipLayer *layer, float *wr);

/* Full layer on device buffers: x [T x d] -> out [T x d] (overwritten);
 * probs [T x E] and ids [T x top_k] are optional (NULL = not written).
 * accumulate != 0 adds into out instead (x += MoE(x_norm) decode form). */
int moe_hip_forward_dev(MoeHipLayer *layer, const float *x, int T, float *out,
                        float *probs, int *ids, int accumulate, void *stream);

/* moe_hip_forward_dev without any device allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Every
 * temporary (routing, dispatch, expert activations, partial products,
 * completion counters) lives in a fixed 128 MiB device array of the library,
 * one per GPU, held until the process ends; the layer's weights and the
 * caller's x, out, probs and ids are the only other memory touched.  A call
 * whose temporaries exceed 128 MiB fails with MOE_HIP_ERR_UNSUPPORTED (the
 * message gives the need): at d_model 256, ffn_hidden 1024 that is above
 * about 10k tokens at top-2; the 64-sequence decode layer of d_model 512,
 * ffn_hidden 2048, E=16 takes 4.2 MB.  The library must be initialised
 * (moe_hip_init or a layer created) on the calling device first.  All calls
 * on one GPU share its array and each call keeps it until the next: calls
 * that overlap on one GPU (two streams, two threads) race. */
int moe_hip_forward_dev_noalloc(MoeHipLayer *layer, const float *x, int T, float *out,
                                float *probs, int *ids, int accumulate, void *stream);

/* The layer forward on T host rows: x [T x d_model] and out [T x d_model]
 * in host memory (pageable), probs [T x E] and ids [T x top_k] too when not
 * null, weights resident in the layer.  The rows go up and the results come
 * back through pinned staging buffers, the copies overlapping each other and,
 * for probs and ids, the expert products; synchronous at return.  This is
 * moe_forward's data movement for callers that keep their weights resident
 * (no counterpart in the reference). */
int moe_hip_forward_host(MoeHipLayer *layer, const float *x, int T, float *out, float *probs,
                         int *ids);

/* rms_norm (src/matrix.c:666-711) on device rows: y [rows x cols] =
 * (x * inv_rms) * w with the reference's summation order and fused
 * multiply-adds, and a correctly rounded 1/sqrt (see moe_block_ffn). */
int moe_hip_rms_norm_dev(const float *x, const float *w, float eps, int rows, int cols,
                         float *y, void *stream);

/* Backward pass of the layer on device rows x [T x d] (no counterpart in
 * the reference: its block backward, src/transformer.c:975-1013, skips the
 * FFN/MoE half).  Gradients of L = sum(dout * out) + aux_coef * aux with
 * out = moe_forward(x) (src/transformer.c:287-366) and the routing held as
 * that forward decides it (recomputed here, bit-exact), where aux is the
 * load-balancing loss src/transformer.c:280-282 describes:
 * aux = n_experts * sum_e f_e * P_e, f_e = (assignments to e) / (T * top_k)
 * (a count: no gradient), P_e = mean over tokens of probs[t][e].
 * Outputs, device, in the weights' layout: dx [T x d], dw_router [d x E],
 * dw_gate, dw_up [n_experts][d x ffn_hidden], dw_down [n_experts][ffn_hidden
 * x d]; accumulate != 0 adds to them.  aux_loss (device float, may be NULL)
 * receives aux.  A router bias, if set, enters the forward but gets no
 * gradient here.  Deterministic; fp32 with fixed summation orders.  Layers
 * of n_experts <= 256 and top_k <= 16 (MOE_HIP_ERR_UNSUPPORTED past them). */
int moe_hip_backward_dev(MoeHipLayer *layer, const float *x, int T, const float *dout,
                         float aux_coef, float *dx, float *dw_router, float *dw_gate,
                         float *dw_up, float *dw_down, float *aux_loss, int accumulate,
                         void *stream);

/* The MoE block's FFN sublayer on a device-resident residual stream x
 * [T x d], in place: x += MoE(rms_norm(x; rms_w, eps)) (src/transformer.c:
 * 760-767 with the residual add of :767; also the decode form of
 * src/inference.c:310-343 for T rows).  x_norm [T x d] receives the
 * normalised rows (NULL: library workspace); probs and ids as in
 * moe_hip_forward_dev.  No host round trip. */
int moe_hip_ffn_sublayer_dev(MoeHipLayer *layer, float *x, const float *rms_w, float eps, int T,
                             float *x_norm, float *probs, int *ids, void *stream);

/* Routing and dispatch only: probs [T x E], ids [T x k], gate weights
 * gw [T x k] (renormalised), counts [E], offsets [E+1], perm [T x k]
 * (perm[pos] = t*k + slot, stable by expert).  Any output may be NULL. */
int moe_hip_route_dev(MoeHipLayer *layer, const float *x, int T, float *probs,
                      int *ids, float *gw, int *counts, int *offsets, int *perm,
                      void *stream);

/* ---------------------------------------------------------------------------
 * The attention half of the KV-cache decode step (src/inference.c:252-308)
 * on the GPU, for B sequences at once, each at its own position.
 * ------------------------------------------------------------------------- */
typedef struct MoeHipAttn MoeHipAttn;

/* One block's attention: n_heads query heads, n_kv_heads kv heads of
 * head_dim (<= 64, multiple of 8, at most 8 query heads per kv head),
 * positions < max_seq_len. */
int moe_hip_attn_create(int d_model, int n_heads, int n_kv_heads, int head_dim, int max_seq_len,
                        MoeHipAttn **attn);
int moe_hip_attn_destroy(MoeHipAttn *attn);
/* Host weights in the reference layout (src/attention.c:133-144): W_Q
 * [d x nh*hd], W_K and W_V [d x nkv*hd], W_O [nh*hd x d]; rms_attn [d]. */
int moe_hip_attn_load(MoeHipAttn *attn, const float *wq, const float *wk, const float *wv,
                      const float *wo, const float *rms_attn);
/* The model's RoPE tables (RoPEBuffer, src/attention.c:151-167): cos and
 * sin [max_seq_len x head_dim/2], host pointers. */
int moe_hip_attn_set_rope(MoeHipAttn *attn, const float *cos_table, const float *sin_table);

/* x [B x d] device residual rows, in place: x += W_O . GQA(RoPE(q), cache)
 * with q, k, v = rms_norm(x; rms_attn, eps) . W_Q, W_K, W_V; k and v are
 * written at row pos[b] of sequence b's caches k_cache, v_cache
 * [B][max_seq_len][nkv*hd] (a LayerKVCache per sequence, contiguous), and
 * head h attends positions 0 .. pos[b] of kv head h / (nh/nkv)
 * (src/inference.c:252-308).  pos: device ints.  The projections are
 * 16 x 16 output tiles with rms_norm's row scale applied after the
 * reduction, and the softmax and V sums run in 128-position chunks, so
 * results match the reference within the layer tolerance rather than bit
 * for bit (deterministically).  Three launches (four for head shapes other
 * than head_dim 16/32/64 with 2, 4 or 8 query heads per kv head).
 * A pos[b] outside [0, max_seq_len) leaves sequence b's caches and x row
 * unchanged. */
int moe_hip_attn_decode_dev(MoeHipAttn *attn, float *x, int B, const int *pos, float *k_cache,
                            float *v_cache, float eps, void *stream);

/* One decoder block of the KV-cache decode step for B sequences
 * (src/inference.c:245-345), on device rows x [B x d] in place:
 * x += Attn(rms_norm(x; rms_attn)) as moe_hip_attn_decode_dev, then
 * x += MoE(rms_norm(x; rms_ffn, eps)) as moe_hip_ffn_sublayer_dev with the
 * layer (same d_model).  The FFN half applies to every row (a pos[b] out
 * of range skips only the attention half).  rms_ffn: device [d]; x_norm
 * [B x d] receives the FFN's normalised rows, bit-identical to
 * moe_hip_rms_norm_dev of the updated x (NULL: library workspace); ids
 * [B x top_k] the expert ids (may be NULL).  The MoE router normalises
 * the rows itself as its first step (a separate rms_norm launch where it
 * cannot). */
int moe_hip_decode_block_dev(MoeHipAttn *attn, MoeHipLayer *layer, const float *rms_ffn, float *x,
                             int B, const int *pos, float *k_cache, float *v_cache, float eps,
                             float *x_norm, int *ids, void *stream);

/* ---------------------------------------------------------------------------
 * Checkpoints: the MoE blocks of a file written by model_save
 * (src/transformer.c:573-616, read back by model_load :624-700) straight into
 * packed device layers, one matrix at a time (host memory: 3 x d x F floats
 * of pinned staging), with every block's rms_ffn scale on the device.
 * Embeddings, attention, dense FFN blocks and the head are skipped.  Every
 * block is MoE when n_experts > 1 (src/transformer.c:437), else none is.
 * ------------------------------------------------------------------------- */
typedef struct MoeHipModel MoeHipModel;

int moe_hip_model_load(const char *path, MoeHipModel **model);
int moe_hip_model_free(MoeHipModel *model);
int moe_hip_model_config(const MoeHipModel *model, ModelConfig *cfg);
/* Block l's MoE layer (owned by the model), or NULL for a dense block. */
MoeHipLayer *moe_hip_model_layer(MoeHipModel *model, int layer);
/* Block l's rms_ffn scale [d_model] in device memory. */
const float *moe_hip_model_rms_ffn(const MoeHipModel *model, int layer);

/* Device synthetic fill: dst[i] = N(mean, std) sample of (seed, stream, i). */
int moe_hip_fill_normal_dev(float *dst, size_t n, uint64_t seed,
                            uint64_t stream_id, float mean, float std,
                            void *stream);

/* Expert-product kernels: 0 = automatic (skinny decode GEMVs when the
 * average expert holds at most 16 rows, grouped MFMA GEMMs otherwise),
 * 1 = always grouped GEMMs, 2 = always decode GEMVs (gate/up fused with a
 * split-K down projection while its partials fit 32 MB, else as 3),
 * 3 = always decode GEMVs as separate gate/up and down launches.  Modes 2
 * and 3 need ffn_hidden % 64 == 0 and T * top_k <= 4096.  Process-wide;
 * every path computes the same layer. */
int moe_hip_set_expert_path(int mode);

/* Routing kernel selection: 0 = automatic, 1 = token x expert tiles,
 * 2 = 16-token row blocks with every expert in one workgroup, in their own
 * launch.  Automatic routes a decode step of up to 64 tokens (up to 16
 * experts, d_model 256 or 512, finite router weights) inside the fused
 * expert kernel, or inside the few-row kernel when the step holds at most 8
 * assignments, with the row blocks' arithmetic.  The tiles take up to 128
 * experts; with mode 1 a wider layer routes by row blocks.  Process-wide;
 * every choice gives the same bits. */
int moe_hip_set_router_path(int mode);

/* Which kernels the library's last layer forward ran (no
 * counterpart in the reference; for tests and tuning): 1 = router launch and
 * grouped GEMMs, 2 = router launch and the fused decode kernel, 3 = router
 * launch and the two-launch decode, 4 = the fused decode kernel with the
 * routing inside, 5 = router launch and the few-row decode kernel (steps of
 * at most 4 assignments), 6 = the few-row decode kernel with the routing
 * inside (at most 8 assignments); 0 before any forward. */
int moe_hip_last_forward_path(void);

/* Verification hook: y[i] = the device's exp_avx2 lane (which = 0,
 * src/matrix.c:82-116) or glibc-expf restatement (which = 1) of x[i], the two
 * scalar exponentials the routing softmax uses. */
int moe_hip_eval_exp(int which, const float *x, float *y, size_t n, void *stream);

/* Calibration hook for hardware memory counters (no counterpart in the
 * reference): reads `bytes` of device memory at src (a nonzero multiple of
 * 32 MiB) through one load path of the kernels, mode 0 = global-to-LDS DMA
 * (the grouped GEMMs' operand loads), 1 = vector loads, 2 = non-temporal
 * vector loads (the decode weight stream), and writes 1024 per-workgroup
 * sums to out. */
int moe_hip_read_probe(const void *src, size_t bytes, int mode, float *out, void *stream);

/* Host link rate (no counterpart in the reference): one host-to-device and
 * one device-to-host copy of `bytes` between pinned host memory and the
 * device, in GB/s (the rate the host drop-ins' staged copies run at). */
int moe_hip_link_rate(size_t bytes, float *h2d_gbs, float *d2h_gbs);

/* Kernel timing of the last moe_hip_forward_dev call on the library's
 * events: milliseconds for [route, dispatch, gate_up, down, combine]. */
int moe_hip_last_timings(float *ms5);
int moe_hip_set_timing(int on);

/* Elapsed device time on the library stream between timer_start and
 * timer_stop (which waits for the stream), in milliseconds. */
int moe_hip_timer_start(void);
int moe_hip_timer_stop(float *ms);
/* Mark i (0 <= i < 64) recorded on the library stream without waiting, and
 * the device time between marks i and j (waits for mark j): per-call times
 * of a loop that is not synchronised inside. */
int moe_hip_timer_mark(int i);
int moe_hip_timer_between(int i, int j, float *ms);

/* ---------------------------------------------------------------------------
 * Device memory helpers for callers with no HIP binding of their own (the
 * Python tests and benchmark use these).  Copies and memsets run on the
 * library stream and are complete at return.  kind: 1 host->device,
 * 2 device->host, 3 device->device.
 * ------------------------------------------------------------------------- */
int moe_hip_dev_alloc(void **ptr, size_t bytes);
int moe_hip_dev_free(void *ptr);
int moe_hip_memcpy(void *dst, const void *src, size_t bytes, int kind);
int moe_hip_memset(void *ptr, int value, size_t bytes);
int moe_hip_synchronize(void);

/* HIP graphs for such callers (the benchmark replays a captured decode
 * step).  graph_begin starts capturing `stream` (NULL: the library stream):
 * work queued on it until graph_end is recorded, not run.  graph_end
 * instantiates the recording into *graph.  Recorded calls must not allocate:
 * run each once beforehand so the library workspace is already sized.  A
 * graph keeps the workspace addresses it recorded, so while any graph made
 * by graph_end is alive, during a capture, and for the rest of the process
 * once a call was recorded into a capture the caller began on its own stream,
 * a call that would grow the workspace fails with MOE_HIP_ERR_ARG instead
 * (moe_hip_forward_dev_noalloc never grows anything). */
int moe_hip_graph_begin(void *stream);
int moe_hip_graph_end(void *stream, void **graph);
int moe_hip_graph_launch(void *graph, void *stream);
int moe_hip_graph_destroy(void *graph);

#ifdef __cplusplus
}
#endif
#endif /* MOE_HIP_H */
