// Internal declarations shared by the yvmoe HIP translation units (gfx950 only).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include "../../include/yvmoe.h"

namespace yvmoe {

// ---------------------------------------------------------------- error reporting
void set_error(const char* fmt, ...);
void clear_error();

#define YV_REQUIRE(cond, code, ...)          \
    do {                                     \
        if (!(cond)) {                       \
            ::yvmoe::set_error(__VA_ARGS__); \
            return (code);                   \
        }                                    \
    } while (0)

#define YV_LAUNCH_CHECK(name)                                                          \
    do {                                                                               \
        hipError_t e_ = hipGetLastError();                                             \
        if (e_ != hipSuccess) {                                                        \
            ::yvmoe::set_error("%s launch failed: %s", name, hipGetErrorString(e_));   \
            return YVMOE_ERR_LAUNCH;                                                   \
        }                                                                              \
    } while (0)

// ---------------------------------------------------------------- sizes
constexpr int kTokPerBlock = 64;  // tokens per routing block
constexpr int kTileRows = 64;     // rows per expert GEMM tile (4 MFMA row blocks)
constexpr int kPredDim = YVMOE_PREDICTOR_DIM;

inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
inline int ceil_div(int a, int b) { return (a + b - 1) / b; }
inline int pad16(int e) { return (e + 15) / 16 * 16; }

// Router output row stride for an activation dtype.
inline int router_ld(int E, int act) {
    return pad16(E) + (act == YVMOE_ACT_BF16 ? 3 * kPredDim : kPredDim);
}

// K splits of the router GEMM: enough work-groups to spread a small batch over the chip,
// at least 128 of K per split (2 k-steps); partial sums are reduced in split order.
// Batches of up to kSmallRouteTok tokens take the two-kernel small-batch routing path
// (per-token top-k with the router's split-K reduction folded in, then everything else in
// one work-group).
constexpr int kSmallRouteTok = 256;
// Most router split partial sums the multi-block top-k kernel adds itself (above
// kSmallRouteTok tokens); more splits are reduced by a launch of their own first.
constexpr int kFoldSplits = 4;

#ifndef YV_ROUTER_KS_MAX
// most router K splits: 16 measured best for 1-256 tokens at H = 4096, E = 64 (cfg2 decode
// layer step 227 -> 224 us against 32 splits; 8 and 4 slower)
#define YV_ROUTER_KS_MAX 16
#endif

// Router GEMMs of more than kSmallRouteTok tokens with bf16 operands run on the LDS-tiled MFMA
// form: 256 x 256 output tiles (the last column block may be partial), K split so that the
// (tile, column block, split) items spread over the 256 CUs.
inline bool router_tiled(int act, int N, int ncols, int K) {
    return act == YVMOE_ACT_BF16 && N > kSmallRouteTok && ncols % 16 == 0 && K % 64 == 0 && K > 0;
}

// k-steps (of 64) per split of the tiled router GEMM: the choice with the least estimated time,
// counted in tile k-steps: rounds of 256 items (one work-group per CU) times k-steps per split,
// plus, when split, the partial sums' extra HBM traffic (ks arrays of N x ncols fp32 written
// by the GEMM and read back by the reduction) at 8 MB per k-step. At most 16 splits.
inline int router_tiled_steps(int N, int ncols, int K) {
    const int units = ceil_div(N, 256) * ceil_div(ncols, 256);
    const int nks = K / 64;
    const double arr = (double)N * ncols * 4 / 8.0e6;
    int best = nks;
    double best_t = (double)ceil_div(units, 256) * nks;
    for (int steps = nks - 1; steps >= 1; --steps) {
        const int ks = ceil_div(nks, steps);
        if (ks > 16) break;
        const double t = (double)ceil_div(units * ks, 256) * steps + 2.0 * ks * arr;
        if (t < best_t) {
            best = steps;
            best_t = t;
        }
    }
    return best;
}

inline int router_ksplit(int N, int E, int act, int H) {
    const int ld = router_ld(E, act);
    if (router_tiled(act, N, ld, H)) return ceil_div(H / 64, router_tiled_steps(N, ld, H));
    const int groups = ceil_div(router_ld(E, act), 64);
    const int wgs = ceil_div(N > 0 ? N : 1, 64) * groups;
    int ks = 1;
    while (ks * 2 <= YV_ROUTER_KS_MAX && wgs * ks * 2 <= 512 && H % (ks * 2 * 64) == 0 &&
           H / (ks * 2) >= 128)
        ks *= 2;
    return ks;
}

// Dense fp32-output GEMMs of more than 64 rows with bf16 operands, 256-multiple columns and
// 64-multiple K run on the LDS-tiled MFMA form (256 x 256 output tiles, no K split).
inline bool dense_tiled(int act, int N, int ncols, int K) {
    return act == YVMOE_ACT_BF16 && N > 64 && ncols % 256 == 0 && K % 64 == 0;
}

// K splits of a dense fp32-output GEMM over ncols columns (same rule as the router's).
inline int dense_ksplit(int N, int ncols, int K) {
    const int wgs = ceil_div(N > 0 ? N : 1, 64) * ceil_div(ncols, 64);
    int ks = 1;
    while (wgs * ks * 2 <= 512 && K % (ks * 2 * 64) == 0 && K / (ks * 2) >= 128) ks *= 2;
    return ks;
}

// Dense fp32-output GEMMs of up to 64 rows with bf16 operands run on the weight-streaming
// form (one 16- or 64-row tile, 64 columns per work-group), K split in two when that keeps
// the work-groups at or below 1024: the weights are read once, the two partial sums are
// summed by the consumer.
inline bool dense_streamed(int act, int N, int ncols, int K) {
    return act == YVMOE_ACT_BF16 && N <= 64 && ncols % 16 == 0 && K % 64 == 0;
}
inline int dense_splits(int act, int N, int ncols, int K) {
    if (dense_tiled(act, N, ncols, K)) return 1;
    if (!dense_streamed(act, N, ncols, K)) return dense_ksplit(N, ncols, K);
    const int items = ceil_div(ncols, 64);
    int ks = 1;
    while (ks < 2 && items * ks * 2 <= 1024 && K % (ks * 2 * 64) == 0 && K / (ks * 2) >= 256) ks *= 2;
    return ks;
}

inline size_t router_partials_bytes(int N, int E, int act, int H) {
    const int ks = router_ksplit(N, E, act, H);
    return ks > 1 ? align_up((size_t)ks * N * router_ld(E, act) * 4, 256) : 0;
}

// Upper bound on the number of GEMM tiles of tile_rows rows over all segments.
inline int max_tiles(int N, int k, int E, int S, int tile_rows) {
    return ceil_div(N * k, tile_rows) + E + S * ceil_div(N, tile_rows);
}

// Workspace layout. The routing region depends on (N, E, k) only; the FFN region follows
// it, so every entry that runs the expert FFN finds its region at the same offset. The FFN
// reads nothing of the routing region: its inputs are the routing's offsets and perm.
struct RouteWs {
    size_t topp, w0, allowed, blockhist, blockoff, blocksum, score, bytes;
};
struct FfnWs {
    size_t seg, tile_seg, tile_row0, ntiles, lseg, lrow0, lntiles, h, bytes;
};

inline RouteWs route_ws(int N, int E, int k) {
    RouteWs w{};
    const int nb = ceil_div(N, kTokPerBlock) > 0 ? ceil_div(N, kTokPerBlock) : 1;
    size_t o = 0;
    const size_t nk = (size_t)N * k;
    w.topp = o;      o = align_up(o + nk * 4, 256);
    w.w0 = o;        o = align_up(o + nk * 4, 256);
    w.allowed = o;   o = align_up(o + nk, 256);
    w.blockhist = o; o = align_up(o + (size_t)nb * E * 4, 256);
    w.blockoff = o;  o = align_up(o + (size_t)nb * E * 4, 256);
    w.blocksum = o;  o = align_up(o + (size_t)nb * 4, 256);
    w.score = o;     o = align_up(o + (size_t)N * 4, 256);
    w.bytes = o;
    return w;
}

inline FfnWs ffn_ws(int N, int k, int E, int S, int F, int act) {
    FfnWs w{};
    const size_t R = (size_t)N * k + (size_t)S * N;
    const int T = max_tiles(N, k, E, S, 16);  // 16-row tiles give the most tiles
    size_t o = 0;
    w.seg = o;       o = align_up(o + (size_t)(E + S + 1) * 4, 256);
    w.tile_seg = o;  o = align_up(o + (size_t)T * 4 + 4, 256);
    w.tile_row0 = o; o = align_up(o + (size_t)T * 4 + 4, 256);
    w.ntiles = o;    o = align_up(o + 4, 256);
    w.lseg = o;      o = align_up(o + (size_t)(E + S) * 4 + 4, 256);  // light tiles (one per segment)
    w.lrow0 = o;     o = align_up(o + (size_t)(E + S) * 4 + 4, 256);
    w.lntiles = o;   o = align_up(o + 4, 256);
    const size_t esz = act == YVMOE_ACT_BF16 ? 2 : 4;
    w.h = o;         o = align_up(o + R * (size_t)F * esz, 256);
    w.bytes = o;
    return w;
}

// Expert output rows [N*k + S*N][H] (yvmoe_forward keeps them in its workspace).
inline size_t y_bytes(int N, int k, int S, int H, int act) {
    const size_t R = (size_t)N * k + (size_t)S * N;
    return align_up(R * (size_t)H * (act == YVMOE_ACT_BF16 ? 2 : 4), 256);
}

// Workspace of yvmoe_dispatch (k = slots per token, routed experts only): the routing region
// (block histograms and offsets), the FFN region after it (where expert_ffn_launch looks for
// it), the expert outputs, then fp32 routing weights, the permutation and its inverse, counts,
// offsets and two scalars (capacity, invalid-slot count).
struct DispatchWs {
    size_t y, w32, perm, pos, counts, offsets, misc, bytes;
};
inline DispatchWs dispatch_ws(int N, int k, int E, int H, int F, int act) {
    DispatchWs w{};
    const size_t nk = (size_t)N * k;
    size_t o = route_ws(N, E, k).bytes + ffn_ws(N, k, E, 0, F, act).bytes;
    w.y = o;       o += y_bytes(N, k, 0, H, act);
    w.w32 = o;     o = align_up(o + nk * 4, 256);
    w.perm = o;    o = align_up(o + nk * 4, 256);
    w.pos = o;     o = align_up(o + nk * 4, 256);
    w.counts = o;  o = align_up(o + (size_t)E * 4, 256);
    w.offsets = o; o = align_up(o + (size_t)(E + 1) * 4, 256);
    w.misc = o;    o = align_up(o + 2 * 4, 256);
    w.bytes = o;
    return w;
}

// ---------------------------------------------------------------- launchers
// Tile table of the expert GEMMs (segments = E routed experts, then S shared experts of N
// rows each; every segment cut into tile_rows-row tiles), in the FFN workspace region. With
// fold > 0 a segment's remainder of at most fold rows joins its last full tile (which then
// holds tile_rows + remainder rows) instead of taking a tile of its own. With light > 0 a
// remainder of at most light rows that is not folded takes no tile of the main table but one of
// the light table (ltile_seg, ltile_row0, lntiles: at most one per segment), which the
// weight-streaming GEMM form runs with light-row tiles (32 or 64).
struct TileTable {
    int* seg;
    int* tile_seg;
    int* tile_row0;
    int* ntiles;
    int S;
    int tile_rows;
    int fold;
    int light;
    int* ltile_seg;
    int* ltile_row0;
    int* lntiles;
};

// Rows the LDS-tiled GEMM form can take beyond its 256-row tile: an expert's remainder of up
// to this many rows is folded into its last full tile.
constexpr int kTileFold = 32;

// Tiles of a segment of `rows` rows in the main table (the rule both tile-table builders
// follow), and whether its remainder takes a light tile instead.
// A remainder (rows past the segment's full tiles) is folded into the last full tile when it
// holds at most fold rows (and there is a full tile), else it takes a light tile when it holds
// at most light rows, else a tile of its own.
__host__ __device__ inline bool seg_folds(int rows, int tile_rows, int fold) {
    const int n = rows / tile_rows, rem = rows - n * tile_rows;
    return rem > 0 && n > 0 && rem <= fold;
}
__host__ __device__ inline int seg_light(int rows, int tile_rows, int fold, int light) {
    const int rem = rows % tile_rows;
    return (rem > 0 && rem <= light && !seg_folds(rows, tile_rows, fold)) ? 1 : 0;
}
__host__ __device__ inline int seg_tiles(int rows, int tile_rows, int fold, int light = 0) {
    const int n = rows / tile_rows, rem = rows - n * tile_rows;
    return n + ((rem > 0 && !seg_folds(rows, tile_rows, fold) && !seg_light(rows, tile_rows, fold, light)) ? 1 : 0);
}

// Whether, and up to how many rows, the LDS-tiled expert GEMMs send remainders to the
// weight-streaming form (light tiles of 32 or 64 rows, the light value): when experts hold few
// tiles each (a mean under two 256-row tiles). A 256-row tile that holds a few dozen rows still
// streams and dequantizes the expert's weights through LDS, at about half the cost of a full
// tile; the streaming form reads them once from HBM with no LDS round trip for the weights.
// Without folding: remainders of at most 32 rows (cfg5 FFN, one box: 256-row tiles only
// 7.62-7.65 ms; light tiles of 16, 32, 64 rows 7.45-7.50, 7.19-7.21, 7.37 ms). With folding
// (remainders of at most kTileFold rows join their last full tile): the remainders of
// kTileFold + 1 .. 64 rows.
inline int tile_light(int N, int k, int E, int fold) {
    const long long mean = (long long)N * k / (E > 0 ? E : 1);
    if (mean >= 512) return 0;
    return fold > 0 ? 64 : 32;
}

// Whether the LDS-tiled expert GEMMs fold remainders: when the mean expert holds one tile and
// at most 2 kTileFold rows more, most experts end a few rows past their first tile, and a
// folded remainder costs an eighth of a tile where a tile of its own costs about half of one.
// Otherwise the tiles run the form without folded rows, which is a few percent faster per tile.
inline int tile_fold(int N, int k, int E) {
    const long long mean = (long long)N * k / (E > 0 ? E : 1);
    return (mean > 256 && mean <= 256 + 2 * kTileFold) ? kTileFold : 0;
}

// YvMoEGate loss inputs (the per-work-group sums of the per-token kernels) for the kernel that
// reduces them (yvmoe_gate_loss.h): the loss kernel, or the small-batch routing kernel when it
// runs next on the stream.
struct GateLossArgs {
    const float* part;  // [E + 2][G]
    int G, E, N;
    float lb_alpha, z_alpha, budget, cap_loss;
    int has_soft;
    float* loss;
};
// The YvMoEGate per-token kernel's own top-k (decode sizes, at most 64 experts): the per-slot
// outputs of route_topk_small_kernel, in the routing workspace and indices.
struct GateTopk {
    int64_t* idx;
    float* topp;
    float* w0;
    int k;
};

// routing (yvmoe_route.hip). Logits (and predictor columns) are the in-order sum of ksplit
// partial copies split_stride floats apart (ksplit = 1: plain logits). With tiles non-null
// (small batches only) the tile table is built as well.
// topk_ready (small batches in fixed-shape mode): the per-token top-k outputs are already in
// place (the YvMoEGate per-token kernel wrote them), so only route_small_kernel runs; with
// loss set (small batches) that kernel also reduces the YvMoEGate loss.
int route_launch(const float* logits, int ld, const float* pred, int pred_ld, int N,
                 const yvmoe_router* r, int cap_override, yvmoe_routing* out, char* ws,
                 hipStream_t st, int ksplit = 1, long long split_stride = 0,
                 const TileTable* tiles = nullptr, bool topk_ready = false,
                 const GateLossArgs* loss = nullptr);
// The per-slot top-k outputs of route_launch's small-batch path for this routing (where
// route_topk_small_kernel writes them).
GateTopk route_topk_outputs(int N, int E, int k, yvmoe_routing* out, char* ws);
// Whether route_launch takes the small-batch path (route_small_kernel) for a fixed-shape
// routing of N tokens.
inline bool route_small_fixed(int N) { return N > 0 && N <= kSmallRouteTok; }
// external routing of the dispatch entry (yvmoe_route.hip): counts, offsets, the stable
// permutation and its inverse (pos = -1 for ids outside [0, E)), the invalid-slot count, and
// with w32 set the bf16 weights widened to fp32.
int dispatch_route_launch(const int64_t* idx, const unsigned short* w_bf16, float* w32, int N,
                          int E, int k, int* counts, int* offsets, int* perm, int* pos,
                          int* invalid, int* cap_scratch, char* ws, hipStream_t st);
// GEMMs and combine (yvmoe_gemm.hip). With reduce = false the router GEMM leaves its split-K
// partial sums in partials (when it splits) for the routing kernel to reduce.
int router_gemm_launch(const void* x, int act, int N, const yvmoe_router* r, float* out,
                       int ld, float* partials, hipStream_t st, bool reduce = true);
// Rows per tile of the expert GEMMs for this batch and layer, and the tile table's location
// in the workspace.
int ffn_tile_rows(int act, int N, int k, int E, int H, int F, int wf);
TileTable ffn_tile_table(int N, int k, int E, int S, int F, int act, int tile_rows, char* ws);
int expert_ffn_launch(const void* x, int act, int N, int k, const yvmoe_expert_weights* w,
                      const yvmoe_routing* routing, void* y, char* ws, hipStream_t st,
                      bool tiles_ready = false);
// out[N][ld] (fp32) = x[N][K] · wᵀ, w [ncols][K] in the activation dtype; split-K partial
// sums (when the rule splits) go to partials and are reduced in split order.
int dense_gemm_launch(const void* x, int act, int N, int K, const void* w, int ncols, float* out,
                      int ld, float* partials, hipStream_t st, const char* name);
// The same product left as dense_splits(act, N, ncols, K) partial sums: split z at
// out + z * N * ld (its K range z * K / splits ...), for the consumer to sum in split order;
// split 0 also adds col_bias[n] to columns n < col_bias_n (col_bias may be NULL).
int dense_partials_launch(const void* x, int act, int N, int K, const void* w, int ncols,
                          float* out, int ld, const float* col_bias, int col_bias_n,
                          hipStream_t st, const char* name);
// YvMoEGate logits and loss (yvmoe_moegate.hip). Workspace: the projections [N][P] (DG
// activations, then the heads), split-K partial sums, per-work-group loss sums.
struct GateWs {
    size_t proj, loss, bytes;
    int groups;
};
int moegate_heads_rows(const yvmoe_moegate* g);
int moegate_proj_rows(const yvmoe_moegate* g);
GateWs gate_ws(int N, int act, const yvmoe_moegate* g);
// topk (optional): the per-token kernel also runs each token's top-k (E <= 64 and the
// work-group-per-token form only; returns whether it did). defer_loss (optional): the loss
// reduction is not launched; its arguments are returned for the caller's next kernel.
int moegate_launch(const void* x, int act, int N, const yvmoe_moegate* g, const int* modal_id,
                   float* logits, float* loss, char* ws, hipStream_t st,
                   const GateTopk* topk = nullptr, bool* topk_done = nullptr,
                   GateLossArgs* defer_loss = nullptr);
// RMSNorm (yvmoe_norm.hip): nn (1 or 2) norms in sequence, one wavefront per row; y may alias x.
struct NormChain {
    const void* w[2];
    const void* b[2];
    float eps[2];
};
int rmsnorm_launch(const void* x, int act, int N, int H, const NormChain& nc, int nn, void* y,
                   hipStream_t st);
int combine_launch(const void* y, int act, int N, int H, int k, int S,
                   const yvmoe_routing* routing, const float* mix, const void* skip,
                   void* out, void* shared_out, hipStream_t st);

}  // namespace yvmoe
