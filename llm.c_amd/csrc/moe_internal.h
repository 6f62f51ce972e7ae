// moe_internal.h — shared declarations between the HIP kernel files and the
// C-ABI layer of libmoe_hip.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace moe {

// Rows per m-tile of the grouped expert GEMMs; the dispatch kernel builds the
// per-expert tile schedule with the same value.
constexpr int kGemmBM = 128;
// Largest expert count the routing kernels support (LDS sizing).
constexpr int kMaxExperts = 256;
// Largest top-k the routing kernels support.
constexpr int kMaxTopK = 16;

struct RouteArgs {
    const float *x;      // [T x d]
    const float *wr;     // [d x E], reference layout
    const float *bias;   // [E] or nullptr
    int T, d, E, k;
    float *probs;        // [T x E]
    int *ids;            // [T x k]
    float *gw;           // [T x k]
    // Row-block router; the tile router runs when wrT is null.
    const float *wrT;    // [E x d], transpose of wr
    int wr_nonfinite;    // wr holds an inf or NaN: apply the zero-skip per step
    int no_dispatch;     // routing only (the decode kernels find their own slots)
    // Optional: the rows are rms_norm(x_raw; rms_w, rms_eps) (rms_rcp =
    // 1/d), computed first into xn_out (== x) by the router itself.
    const float *x_raw = nullptr;
    const float *rms_w = nullptr;
    float rms_eps = 0.0f, rms_rcp = 0.0f;
    float *xn_out = nullptr;
};

// Up to this many 16-token row blocks the row-block router's last workgroup
// performs the dispatch itself.
constexpr int kRowsFusedMaxBlocks = 256;

struct DispatchArgs {
    const int *ids;      // [T x k]
    int n;               // T * k
    int E;
    int bm;              // rows per m-tile for the schedule
    int *counts;         // [E]
    int *offsets;        // [E + 1]
    int *tile_off;       // [E + 1] m-tile prefix; tile_off[E] = total m-tiles
    int *perm;           // [n]
    int *counter;        // zeroed device int for the fused path (reset after use)
    int *tile_expert;    // [n / bm + E] expert of each m-tile (optional)
    int *wide = nullptr; // [wide_dispatch_ints(n, E)] (layers routed by route_wide.hip)
};

// Up to this many (token, slot) assignments, and router workgroups, the
// router's last workgroup performs the dispatch itself.
constexpr int kFusedDispatchMax = 4096;
constexpr int kFusedDispatchMaxBlocks = 16;

struct GemmArgs {
    // A rows: gate/up gathers x[perm[pos] / k]; down reads H[pos].
    const float *a;      // x [T x K] (gate/up) or H [n x K] (down)
    const int *perm;     // [n]
    int topk;            // k, to turn perm entries into tokens
    const float *b;      // packed weights, [E][N][K] (K contiguous)
    float *c;            // H [n x F] (gate/up) or Ys [n x N] indexed by perm (down)
    const int *offsets;  // [E + 1]
    const int *tile_off; // [E + 1]
    const int *tile_expert; // [max_mtiles] expert of each m-tile
    int E;
    int K;               // reduction length
    int N;               // packed output columns (2F for gate/up, d for down)
    int ldc;             // row stride of c (F for gate/up, d for down)
    int max_mtiles;      // grid bound on m-tiles
    // Down projection only: the reduction split ksplit ways (gemm_plan),
    // split s writing its partial to c + s * split_stride.
    int ksplit = 1;
    size_t split_stride = 0;
    // Down projection in stream-K form (down_plan): sk_groups workgroups
    // share the (tile, K slice) units equally; piece s of a tile writes slot
    // s, and pieces[row][n-tile] receives the tile's piece count.
    int streamk = 0;
    int sk_groups = 0;
    int *pieces = nullptr;
    // Backward epilogues: mode 2 also writes H = swiglu(G, U) to c2.
    float *c2 = nullptr;
    int ldc2 = 0;
    // Gate/up with a split tail (gateup_tail_groups): the whole rounds of
    // tail_groups workgroups take whole tiles; the R tiles left over are
    // split along the reduction into S = min(K / 32, 4, tail_groups / R)
    // pieces (when S >= 2), which write their raw gate and up sums to
    // tail_part [R * S][128][256]; launch_gateup_fixup adds the pieces in
    // order and writes H.
    int tail_groups = 0;
    float *tail_part = nullptr;
    // Whole-tile grid in a given m-tile order (order[i] = the i-th m-tile
    // to run; launch_short_first_order), or null for m-tile order.
    const int *order = nullptr;
};

struct CombineArgs {
    const float *ys;     // [ksplit][T*k x d], slot-indexed expert outputs
    const float *gw;     // [T x k]
    float *out;          // [T x d]
    int T, d, k;
    int accumulate;      // out += combined instead of out = combined
    int ksplit;          // partial products per slot (1 for the GEMM path)
    size_t split_stride; // floats between consecutive partials
    // With pieces: slot a's columns [pieces_cols j, pieces_cols (j + 1)) add
    // pieces[a * (d / pieces_cols) + j] partials instead of ksplit.
    const int *pieces = nullptr;
    int pieces_cols = 0;
};

struct DecodeArgs {
    const float *x;      // gate/up: x [T x d]; down: H [n x F]
    const int *ids;      // [n] expert of each assignment a = t*k + slot
    int topk;
    const float *w;      // packed weights (wgu or wdT)
    float *out;          // gate/up: H [n x F]; down: Yp [ksplit][n][d], both by assignment;
                         // fused gate/up + down: Yp [F/64][n][d]
    const float *w2;     // gate/up only: wdT for the fused kernel, or nullptr
    int d, F, E;
    int ksplit;          // down: splits of the F reduction
    int nslots;          // n = T * k
};

// Most assignments (T * k) the decode kernels take (LDS slot list).
constexpr int kDecodeMaxSlots = 4096;
// Largest split-K partial buffer ([F/(16*waves)][T*k][d] floats) the fused
// decode kernel may write; larger layers use the separate down kernel.
constexpr size_t kFusedPartialBytes = (size_t)32 << 20;


hipError_t launch_route_dispatch(const RouteArgs &a, const DispatchArgs &da, hipStream_t s);
// Layers past the fast routing kernels' tables (n_experts > kMaxExperts or
// top_k > kMaxTopK) route through general kernels (route_wide.hip), up to
// these limits; launch_route_dispatch hands them over.  They need
// RouteArgs.probs (the logits go there first) and, with the dispatch,
// DispatchArgs.wide.
constexpr int kWideMaxExperts = 4096, kWideMaxTopK = 256;
bool route_wide_ok(int E, int k);
size_t wide_dispatch_ints(size_t n, int E);
hipError_t launch_route_wide(const RouteArgs &a, const DispatchArgs &da, hipStream_t s);
hipError_t launch_gemm_gateup(const GemmArgs &a, hipStream_t s);
// The split tail's pieces of a gate/up launch with tail_groups > 0 added in
// order, swiglu applied, written to H (same stream, after the gate/up).
hipError_t launch_gateup_fixup(const GemmArgs &a, hipStream_t s);
// The same for a tile-engine launch of mode 0, 2 or 3 (launch_gemm_bwd):
// the pieces' sums go through that mode's epilogue.
hipError_t launch_tail_fixup(const GemmArgs &a, int mode, hipStream_t s);
hipError_t launch_gemm_down(const GemmArgs &a, hipStream_t s);
// order [tile_off[E]] = the experts' short last m-tiles (97 rows or fewer)
// in expert order, then every other m-tile in m-tile order (one workgroup).
hipError_t launch_short_first_order(const int *offsets, const int *tile_off, int E, int *order,
                                    hipStream_t s);
// The backward's tile epilogues (gemm.hip), no reduction split:
//   mode 2  gate/up rows gathered like the forward: c = [G | U] per 32-feature
//           group in the packed column order (ldc = 2F), c2 = H (ldc2 = F);
//   mode 3  a = dY rows, b = the unit transpose of wdT (N = F, K = d): the
//           tile is dH, turned into dG, dU in place over c = [G | U].
hipError_t launch_gemm_bwd(const GemmArgs &a, int mode, hipStream_t s);
// dst[e] = transpose of src[e] in the packed unit layout: src [E][R][C],
// dst [E][C][R] (R, C multiples of 16).
hipError_t launch_transpose_units(const float *src, float *dst, int R, int C, int E,
                                  hipStream_t s);
hipError_t launch_combine(const CombineArgs &a, hipStream_t s);
// Rows of src_cols floats into rows of dst_cols: zero-filled past src_cols,
// or cut to the first dst_cols.
hipError_t launch_copy_rows(const float *src, int rows, int src_cols, float *dst, int dst_cols,
                            hipStream_t s);
hipError_t launch_decode_gateup(const DecodeArgs &a, hipStream_t s);
hipError_t launch_decode_down(const DecodeArgs &a, hipStream_t s);
// The fused decode kernel with the routing inside (every workgroup routes
// all T tokens, then runs its item on the rows it holds): T <= 64, E <= 16,
// d of 256 or 512, F % 128 == 0 (decode_routed_ok).  ra: the routing of the
// same rows (row-block router arguments: wrT, optional bias and rms_norm);
// a: the fused kernel's (out = the split-K partials, w2 = wdT).
bool decode_routed_ok(int T, int d, int F, int E, int k);
hipError_t launch_decode_routed(const DecodeArgs &a, const RouteArgs &ra, hipStream_t s);
// Decode steps with at most kTinySlots assignments (decode_tiny.hip): the
// used experts' 16-feature groups, one workgroup each, writing split-K
// partials Yp [F / 16][n][d] (out; w = wgu, w2 = wdT) that the combine adds
// (ksplit F / 16, at most kTinyMaxGroups).  d of 256, 512 or 1024, F % 32 == 0.
// With ra: every workgroup routes the T tokens itself first (E <= 16, d of
// 256 or 512; ra as for the routed kernel), writing ids, gate weights and
// probabilities through ra.  Steps after a router launch take it up to
// kTinyLaunchSlots assignments, with the routing inside up to kTinySlots.
constexpr int kTinySlots = 8, kTinyLaunchSlots = 4, kTinyMaxGroups = 128;
bool decode_tiny_ok(int n, int d, int F, int E);
bool decode_tiny_routed_ok(int T, int d, int F, int E, int k);
hipError_t launch_decode_tiny(const DecodeArgs &a, const RouteArgs *ra, hipStream_t s);
// Waves per item of the fused decode kernel (8 when d and F allow, else 4);
// its split-K partials number F / (16 * waves).
int decode_fused_waves(int d, int F);
// Number of reduction splits the decode down-projection uses.
int decode_ksplit(int d, int F, int E);

// Weight packing (reference layout -> device layout) and its inverse.
hipError_t launch_pack_gateup(const float *wg, const float *wu, float *dst,
                              int d, int F, hipStream_t s);
hipError_t launch_pack_down(const float *wd, float *dst, int F, int d,
                            hipStream_t s);
hipError_t launch_unpack_gateup(const float *src, float *wg, float *wu, int d,
                                int F, hipStream_t s);
hipError_t launch_unpack_down(const float *src, float *wd, int F, int d,
                              hipStream_t s);
// All E experts at once: wg, wu [E][d x F], wd [E][F x d].
hipError_t launch_unpack_experts(const float *wgu, const float *wdT, float *wg, float *wu,
                                 float *wd, int E, int d, int F, hipStream_t s);
// The attention half of a decode step for B sequences (attention.hip).
struct AttnArgs {
    float *x;               // [B x d] residual stream: x += Attn(rms_norm(x))
    const float *rms_w;     // [d] rms_attn
    float eps;
    const float *wq, *wk, *wv, *wo;   // reference layout: [d x qd], [d x kd] x2, [qd x d]
    const float *cos_t, *sin_t;       // RoPE tables [max_seq x hd/2]
    float *kc, *vc;         // caches [B][max_seq][kd]
    const int *pos;         // [B] position of each sequence's new token
    float *q;               // [B x qd] workspace
    float *o;               // [B x qd] workspace (merged head outputs)
    float *part;            // attn_part_floats(...) workspace: chunk partials
    int *cnt_merge;         // attn_merge_counters(B, nkv) device ints, zero between launches
    int B, d, nh, nkv, hd, qd, kd, max_seq;
    float scale;            // 1 / sqrt(hd)
    // Optional copies packed in 16-column tiles ([N/16][K][16], see
    // launch_pack_cols16): the projection tiles then read one contiguous
    // block per tile.  wqkv_p holds [wq | wk | wv] (K = d), wo_p wo (K = qd).
    const float *wqkv_p = nullptr, *wo_p = nullptr;
};
size_t attn_part_floats(int B, int nh, int hd, int max_seq);
// Merge counters: one per (sequence, kv head).
inline int attn_merge_counters(int B, int nkv) { return B * nkv; }
hipError_t launch_attn_decode(const AttnArgs &a, hipStream_t s);
// Columns col0 .. col0 + N of a K-row matrix packed in 16-column tiles:
// dst[((col0 + c) / 16) K 16 + k 16 + c % 16] = src[k N + c] (col0, N
// multiples of 16).
hipError_t launch_pack_cols16(const float *src, float *dst, int K, int N, int col0,
                              hipStream_t s);

// Backward pass of the layer (backward.hip) with the routing of a forward
// already run (probs, ids, gw, counts, offsets, tile schedule, perm).
// Weights in the reference layout: wr [d x E], wg, wu [E][d x F], wd [E][F x d].
// Workspace: G, U, H [n x F], dH [backward_dh_floats], Y, dY [n x d]
// (n = T k), dgw [n], inv [n], dlogits [T x E].  Outputs (accumulate: added to): dx [T x d], dwr,
// dwg, dwu, dwd (layouts of the weights); aux (optional) = the loss value.
struct BackwardArgs {
    const float *x, *dout;
    const float *wr, *wg, *wu, *wd;
    // Set (backward_engine_ok): the packed wgu, wdT and workspace for their
    // unit transposes [E][d x 2F], [E][F x d]; wg, wu, wd then unused.  G and
    // U must be adjacent (G + n F == U), Y hold backward_slot_splits(...)
    // times [n x d].
    const float *wgu = nullptr, *wdT = nullptr;
    float *wguT = nullptr, *wdTT = nullptr;
    const float *wrT = nullptr;   // [E x d], the router transposed (required)
    const float *probs, *gw;
    const int *ids, *counts, *offsets, *tile_off, *tile_expert, *perm;
    int T, d, F, E, k, max_mtiles;
    float aux_coef;
    float *G, *U, *H, *dH, *Y, *dY, *dgw, *dlogits;
    int *inv;
    int *pieces = nullptr;   // [n][d / 256] when a down_plan is stream-K
    // Split-tail pieces of the GU recompute and dH products (engine path),
    // backward_tail_floats(...) floats, or null for whole tiles only.
    float *tail_part = nullptr;
    float *dx, *dwr, *dwg, *dwu, *dwd, *aux;
    int accumulate;
};
hipError_t launch_moe_backward(const BackwardArgs &b, hipStream_t s);
// The backward runs its row products on the grouped tile engine.
bool backward_engine_ok(int d, int F);
// Partial products per slot row the engine path leaves in Y (1 otherwise);
// n = T * k.
int backward_slot_splits(int d, int F, int max_mtiles, size_t n);
// Floats of BackwardArgs::tail_part the engine path uses (0: none).
size_t backward_tail_floats(int d, int F, int max_mtiles);
// Floats of BackwardArgs::dH: n x F, and at least one row chunk of the
// router gradient's partials (d E + E), which reuse it at the end.
size_t backward_dh_floats(size_t n, int d, int F, int E);

// rms_norm (src/matrix.c:666-711) of rows x cols, weight w [cols].
hipError_t launch_rms_norm(const float *x, const float *w, float eps, int rows, int cols,
                           float *y, hipStream_t s);
// dst[c][r] = src[r][c] for a rows x cols matrix.
hipError_t launch_transpose(const float *src, float *dst, int rows, int cols, hipStream_t s);
// Elementwise exp_poly (which = 0) or glibc-expf (which = 1) on the device,
// exactly as the routing kernels evaluate them.
hipError_t launch_eval_exp(int which, const float *x, float *y, size_t n, hipStream_t s);
// Reads bytes of src through one load path (0 LDS DMA, 1 buffer loads,
// 2 non-temporal buffer loads) and writes 1024 per-workgroup sums to out;
// bytes must be a multiple of 32 MiB.
hipError_t launch_read_probe(const float *src, size_t bytes, int mode, float *out,
                             hipStream_t s);
// p[0 .. n) = 0 by a kernel (safe to record in a graph, unlike a memset node).
hipError_t launch_zero_ints(int *p, int n, hipStream_t s);
// dst = src by a kernel (bytes and both addresses multiples of 16); either
// side may be pinned host memory.
hipError_t launch_copy16(void *dst, const void *src, size_t bytes, hipStream_t s);
hipError_t launch_fill_normal(float *dst, size_t n, uint64_t seed,
                              uint64_t stream_id, float mean, float std,
                              hipStream_t s);

// Tile width (64, 128 or 256 columns) and reduction split of a grouped GEMM
// launch, sized for ~1024 waves in flight (gemm.hip).
struct GemmPlan {
    int bn, ksplit;
};
GemmPlan gemm_plan(int N, int K, int max_mtiles, bool allow_split);

// The forward's down projection: classic (the gemm_plan split) or, for
// grids of a few rounds, stream-K over `groups` workgroups with at most
// `slots` partials per tile.  n: the routed rows (T * k).
struct DownPlan {
    int bn, slots, streamk, groups;
};
DownPlan down_plan(int N, int K, int max_mtiles, size_t n);
// Workgroups per round for a gate/up launch with a split tail (the CUs), or
// 0 for whole tiles only: used when 256-column tiles make fewer than 4
// rounds, where the last, partial round is a large share of the launch.
// The pieces take at most kGemmBM * 256 * groups floats.
int gateup_tail_groups(int N, int K, int max_mtiles);

// Compute units of the current device (cached; 256 on MI355X).
int device_cus();

}  // namespace moe
