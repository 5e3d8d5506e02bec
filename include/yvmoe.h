/*
 * yvmoe.h — C ABI of the MI355X (gfx950) Yv MoE layer inference forward.
 *
 * Every entry point takes raw device pointers and sizes, never allocates or frees device
 * memory, launches only on the stream it is given (a hipStream_t passed as void*), and
 * returns a yvmoe_status. yvmoe_last_error() returns a thread-local message for the last
 * failure on the calling thread. Scratch memory comes from the caller as a workspace whose
 * size yvmoe_workspace_bytes() reports. Activations, outputs and workspaces are read and
 * written in 16-byte vectors: yvmoe_expert_ffn, yvmoe_forward and yvmoe_forward_moegate
 * reject an x, y / out or workspace pointer that is not 16-byte aligned (YVMOE_ERR_ARG).
 *
 * Reference interfaces replaced (Dunimd-Experimental/PiscesLx):
 *   yvmoe_router_logits  -> YvStableMoEGate.gate(x_flat) and complexity_predictor(x)
 *                           model/moe/gate.py:1179, :1112-1117, fixed mode :1148
 *   yvmoe_route          -> YvStableMoEGate.forward after the logits (softmax, topk,
 *                           double softmax, capacity trim) model/moe/gate.py:1147-1241,
 *                           plus the sort / bincount / cumsum of
 *                           PiscesLxFusedMoEDispatch.forward opss/infer/fused_moe.py:69-100
 *   yvmoe_expert_ffn     -> the per-expert loop of PiscesLxFusedMoEDispatch.forward
 *                           opss/infer/fused_moe.py:103-111 calling YvSwiGLUExpert.forward
 *                           model/moe/expert.py:475-489, and the shared experts of
 *                           YvDynamicMoELayer._compute_shared_expert_output
 *                           model/moe/layer.py:812-865
 *   yvmoe_dispatch       -> PiscesLxFusedMoEDispatch.forward opss/infer/fused_moe.py:54-123
 *                           and PiscesLxFusedMoe.fused_moe_dispatch :129-143 (external
 *                           routing weights and expert indices, routed experts, combine)
 *   yvmoe_combine        -> the index_add_ combine opss/infer/fused_moe.py:117-119, the
 *                           routed + shared sum model/moe/layer.py:942-945 and
 *                           _apply_skip_residual model/moe/layer.py:741-753
 *   yvmoe_forward        -> YvDeepSeekMoELayer.forward / YvDynamicMoELayer.forward
 *                           model/moe/layer.py:1283-1396 / :867-963 (inference)
 *   yvmoe_moegate_logits -> YvMoEGate.forward in eval mode up to the top-k (steps 2-8 and the
 *                           loss of step 13), model/moe/gate.py:310-393, :433-444; the top-k
 *                           and its softmax (gate.py:414-416) are yvmoe_route in fixed mode
 *   yvmoe_moegate_forward-> YvMoEGate.forward in eval mode (logits, loss and routing)
 *   yvmoe_forward_moegate-> YvDynamicMoELayer.forward with its YvMoEGate router
 *                           model/moe/layer.py:867-963 (inference)
 *   yvmoe_rmsnorm        -> YvRMSNorm.forward model/core/norms.py:206-208 via
 *                           fused_rms_norm opss/kernels/fused_rms_norm.py:42; two in a
 *                           row = YvHybridBlock's norm_fusion then norm_mlp
 *                           model/core/hybrid.py:1359, :1310
 */
#ifndef YVMOE_H
#define YVMOE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef enum {
    YVMOE_OK = 0,
    YVMOE_ERR_ARG = 1,         /* null pointer or value out of range */
    YVMOE_ERR_SHAPE = 2,       /* sizes the kernels do not support (see limits below) */
    YVMOE_ERR_DTYPE = 3,       /* unknown activation dtype or weight format */
    YVMOE_ERR_UNSUPPORTED = 4, /* gate state the inference path rejects */
    YVMOE_ERR_LAUNCH = 5,      /* a kernel launch failed */
    YVMOE_ERR_WORKSPACE = 6    /* workspace missing or smaller than yvmoe_workspace_bytes */
} yvmoe_status;

/* activation dtype of x, the expert intermediates and the output */
typedef enum { YVMOE_ACT_F32 = 0, YVMOE_ACT_BF16 = 1 } yvmoe_act_dtype;

/* expert weight formats (the values of nn.Linear.weight [out][in] per expert; storage order
 * below, at yvmoe_expert_weights) */
typedef enum {
    YVMOE_W_F32 = 0,  /* fp32 weights, no scales (activations must be fp32) */
    YVMOE_W_BF16 = 1, /* bf16 weights, no scales */
    YVMOE_W_INT8 = 2, /* int8 symmetric per output channel: w = q * s, s bf16 [out] */
    YVMOE_W_INT4 = 3, /* int4, group 128 along in, zero point 8: w = (q - 8) * s,
                         two codes per byte, low nibble = even input index,
                         s bf16 [out][in/128] */
    YVMOE_W_FP8 = 4   /* fp8 e4m3fn (OCP), w = q * s, s fp32 per 128x128 block
                         [out/128][in/128] */
} yvmoe_weight_format;

/* Limits checked on entry: 1 <= E <= 256, 1 <= k <= min(E, 16), 0 <= S <= 8,
 * H and F multiples of 64 (of 128 for INT4 and FP8), N >= 0. */
#define YVMOE_MAX_EXPERTS 256
#define YVMOE_MAX_TOPK 16
#define YVMOE_MAX_SHARED 8
#define YVMOE_PREDICTOR_DIM 64

/*
 * Routed and shared expert weights, stacked: experts [0, E) are the routed experts,
 * [E, E + S) the shared experts (model/moe/layer.py:665-705 keys
 * experts.{e}.{gate,up,down}_proj.weight and shared_experts.{s}.expert.*).
 *   w_gate, w_up : [E+S][F][H] elements of the format (INT4: [E+S][F][H/2] bytes)
 *   w_down       : [E+S][H][F]                         (INT4: [E+S][H][F/2] bytes)
 *   Storage order of w_*: F32 row-major; BF16, INT8, INT4 and FP8 in 16-row x 64-column
 *   blocks, each block contiguous, blocks ordered [out/16][in/64]. Inside a block, piece
 *   (g, r) — row r (0..15), columns 16 g .. 16 g + 15 (g = 0..3) — starts at byte
 *   (16 g + r) * 16 (INT8, FP8: 16 codes; INT4: at (16 g + r) * 8, 8 bytes, low nibble =
 *   even column); BF16 pieces put columns 16 g .. 16 g + 7 at (16 g + r) * 16 and
 *   16 g + 8 .. 16 g + 15 at 1024 + (16 g + r) * 16. Block bytes: 1024 (INT8, FP8), 512
 *   (INT4), 2048 (BF16). pisceslx_amd/quant.py block_matrix() writes this order.
 *   s_gate, s_up : INT8 bf16 [E+S][F]; INT4 bf16 [E+S][F][H/128];
 *                  FP8 fp32 [E+S][F/128][H/128]; NULL otherwise
 *   s_down       : INT8 bf16 [E+S][H]; INT4 bf16 [E+S][H][F/128];
 *                  FP8 fp32 [E+S][H/128][F/128]; NULL otherwise
 */
typedef struct {
    int32_t format; /* yvmoe_weight_format */
    int32_t num_routed;
    int32_t num_shared;
    int32_t hidden;
    int32_t ffn;
    const void* w_gate;
    const void* w_up;
    const void* w_down;
    const void* s_gate;
    const void* s_up;
    const void* s_down;
} yvmoe_expert_weights;

/*
 * Router state of YvStableMoEGate (model/moe/gate.py:895-1028).
 *   w_router : activations bf16 -> bf16 [Ep + 192][H] = [gate.weight padded to Ep rows;
 *              W1 hi; W1 mid; W1 lo], where W1 = complexity_predictor[0].weight [64][H]
 *              split into three bf16 terms whose sum is W1 exactly, stored in the
 *              16 x 64 block order of yvmoe_expert_weights (BF16);
 *              activations fp32 -> fp32 [Ep + 64][H] = [gate.weight padded; W1], row-major.
 *              Ep = E rounded up to a multiple of 16 (padding rows are zero).
 *   b1 [64], w2 [64], b2 [1] : the rest of complexity_predictor (fp32).
 *   bias [E] or NULL : added to the logits before the softmax — expert_bias in
 *              fixed_shape_mode (gate.py:1149), the load adjustment 0.1*(pred - recent)
 *              otherwise (gate.py:1203-1204).
 */
typedef struct {
    int32_t num_experts; /* E */
    int32_t hidden;      /* H */
    int32_t top_k;       /* k */
    int32_t fixed_shape_mode;
    int32_t dynamic_capacity; /* enable_dynamic_capacity */
    int32_t min_capacity;
    double capacity_factor; /* used when dynamic_capacity == 0 */
    const void* w_router;
    const float* b1;
    const float* w2;
    const float* b2;
    const float* bias;
} yvmoe_router;

/*
 * Routing results (device buffers, caller-allocated).
 *   weights [N][k] fp32, indices [N][k] int64 : the gate's (weights, top_idx)
 *   counts [E], offsets [E+1] int32 : bincount and exclusive prefix sum
 *   perm [N*k] int32 : flat slot t*k+j at each expert-sorted position (stable argsort)
 *   pos [N*k] int32  : inverse of perm
 *   capacity [1] int32 : the capacity used (-1 in fixed_shape_mode)
 */
typedef struct {
    float* weights;
    int64_t* indices;
    int32_t* counts;
    int32_t* offsets;
    int32_t* perm;
    int32_t* pos;
    int32_t* capacity;
} yvmoe_routing;

const char* yvmoe_last_error(void);
int32_t yvmoe_version(void);

/* Workspace bytes needed by yvmoe_route / yvmoe_expert_ffn / yvmoe_forward for N tokens. */
size_t yvmoe_workspace_bytes(int32_t n_tokens, int32_t act_dtype, const yvmoe_router* router,
                             const yvmoe_expert_weights* experts);

/*
 * logits_out [N][ld] fp32 with ld = Ep + 192 (bf16 x) or Ep + 64 (fp32 x): columns [0, E)
 * are the gate logits, the rest the complexity predictor's first-layer terms. The values
 * are bit-identical to the logits yvmoe_forward routes on (same split of the K sum, same
 * summation order). workspace: at least yvmoe_router_workspace_bytes() bytes.
 */
size_t yvmoe_router_workspace_bytes(int32_t n_tokens, int32_t act_dtype, const yvmoe_router* router);
int32_t yvmoe_router_logits(const void* x, int32_t act_dtype, int32_t n_tokens,
                            const yvmoe_router* router, float* logits_out, int32_t ld,
                            void* workspace, size_t workspace_bytes, void* stream);

/*
 * Routing from fp32 logits [N][ld] (the first E columns are used).
 *   predictor : NULL, or the predictor columns of yvmoe_router_logits (row stride ld,
 *               column offset Ep) — required when the capacity is dynamic and
 *               capacity_override < 0.
 *   capacity_override >= 0 replaces the computed capacity (ignored in fixed mode).
 */
int32_t yvmoe_route(const float* logits, int32_t ld, const float* predictor, int32_t n_tokens,
                    const yvmoe_router* router, int32_t capacity_override, yvmoe_routing* out,
                    void* workspace, size_t workspace_bytes, void* stream);

/*
 * Grouped SwiGLU FFN of all routed slots and shared experts:
 *   y [N*k + S*N][H] (activation dtype) — rows [0, N*k) in expert-sorted order (the
 *   routing's perm), rows N*k + s*N + t for shared expert s and token t.
 * Reads the routing's offsets and perm only (any workspace of the size
 * yvmoe_workspace_bytes() gives will do: nothing from an earlier call is read from it).
 */
int32_t yvmoe_expert_ffn(const void* x, int32_t act_dtype, int32_t n_tokens, int32_t top_k,
                         const yvmoe_expert_weights* experts, const yvmoe_routing* routing,
                         void* y, void* workspace, size_t workspace_bytes, void* stream);

/*
 * PiscesLxFusedMoEDispatch.forward (opss/infer/fused_moe.py:54-123) from a routing the caller
 * computed with any router: routing_weights [N][k] (fp32 or bf16, weight_dtype = YVMOE_ACT_F32
 * or YVMOE_ACT_BF16) and expert_indices [N][k] int64, k = slots_per_token (the indices' last
 * dimension, fused_moe.py:76-82). On the device: counts = bincount(indices), offsets = their
 * exclusive prefix sum, the stable expert-sorted order (argsort(stable=True), fused_moe.py:87),
 * the grouped SwiGLU FFN of every slot (zero-weight slots included; the routed experts only —
 * experts->num_shared is ignored), then
 *   out[t] = round( sum_j w[t,j] * Y[t,j] )   (fp32, slot order j = 0..k-1, rounded once).
 * A slot whose index lies outside [0, E) is not computed and adds nothing: the kernels never
 * read out of bounds, and *invalid (int32 device scalar, may be NULL) receives the number of
 * such slots so the caller can raise the reference's error. counts [E] / offsets [E+1] (int32,
 * may be NULL) receive the reference's expert_counts / expert_offsets; y_out [N*k][H] (may be
 * NULL) receives the expert outputs in expert-sorted order (for collect_stats). Nothing here
 * synchronizes with the host. workspace: yvmoe_dispatch_workspace_bytes().
 */
size_t yvmoe_dispatch_workspace_bytes(int32_t n_tokens, int32_t act_dtype, int32_t slots_per_token,
                                      const yvmoe_expert_weights* experts);
int32_t yvmoe_dispatch(const void* x, int32_t act_dtype, int32_t n_tokens,
                       const void* routing_weights, int32_t weight_dtype,
                       const int64_t* expert_indices, int32_t slots_per_token,
                       const yvmoe_expert_weights* experts, void* out, void* y_out,
                       int32_t* counts, int32_t* offsets, int32_t* invalid, void* workspace,
                       size_t workspace_bytes, void* stream);

/*
 * out[t] = sum_j weights[t,j] * y[pos[t*k+j]] + shared[t] + 0.1 * skip[t], accumulated in
 * fp32 and rounded once; shared[t] = sum_s mix[s] * y[N*k + s*N + t].
 *   mix [S] fp32 = softmax(shared_expert_weight); skip (activation dtype [N][H]) or NULL;
 *   shared_out [N][H] or NULL receives shared[t] (the next call's skip buffer).
 */
int32_t yvmoe_combine(const void* y, int32_t act_dtype, int32_t n_tokens, int32_t hidden,
                      int32_t top_k, int32_t num_shared, const yvmoe_routing* routing,
                      const float* mix, const void* skip, void* out, void* shared_out,
                      void* stream);

/* The whole layer: router logits, routing, expert FFN and combine. */
int32_t yvmoe_forward(const void* x, int32_t act_dtype, int32_t n_tokens,
                      const yvmoe_router* router, const yvmoe_expert_weights* experts,
                      const float* mix, const void* skip, void* out, void* shared_out,
                      yvmoe_routing* routing, void* workspace, size_t workspace_bytes,
                      void* stream);

/*
 * yvmoe_forward with no workspace argument: the whole layer on a scratch buffer the library
 * holds itself, so the call allocates nothing (no hipMalloc / hipFree, no allocating library
 * routine). This entry point has no counterpart in the reference; it is for callers that
 * cannot allocate device memory: code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc. The caller still passes x, out, shared_out and the routing buffers.
 * The scratch is one device array of YVMOE_STATIC_SCRATCH_BYTES per GPU. It is part of the
 * library's device code, so it is reserved on a GPU when that code is loaded there (at the
 * latest by the first call of any entry point on that GPU, whether or not this one is ever
 * called) and held until the process ends: every process that uses the library pays 64 MiB
 * of device memory per GPU it runs on. A call whose yvmoe_workspace_bytes() exceeds it
 * returns YVMOE_ERR_WORKSPACE (at cfg2's shape, hidden 4096 / 64 experts / top-6 / 2 shared,
 * up to 635 tokens fit). Every call on one GPU shares that GPU's scratch, which keeps the last
 * call's contents: calls that overlap on one GPU (other streams, other host threads) race.
 */
#define YVMOE_STATIC_SCRATCH_BYTES (64u << 20)
int32_t yvmoe_forward_static(const void* x, int32_t act_dtype, int32_t n_tokens,
                             const yvmoe_router* router, const yvmoe_expert_weights* experts,
                             const float* mix, const void* skip, void* out, void* shared_out,
                             yvmoe_routing* routing, void* stream);

/*
 * YvMoEGate (model/moe/gate.py:140-451), the router the reference's MoE layers build
 * (model/moe/layer.py:754-777). Weights as the module holds them, regrouped once:
 *   w_proj [P][H] (activation dtype), the projections of x in one matrix: with the HiCL head,
 *           rows [0, dg_dim) hicl_dg_encoder.dg_proj.weight; then Rh = round_up(4E + D, 256)
 *           head rows: gate.weight, got_cluster_proj.weight, gate_k.weight, gate_v.weight
 *           (E rows each), input_encoder.0.weight (D rows), zero rows.
 *           P = dg_dim + Rh with the HiCL head, Rh without; bf16: in the 16 x 64 block
 *           order of yvmoe_expert_weights (BF16), fp32: row-major;
 *   dg_bias [dg_dim];
 *   prototypes_t [dg_dim][E] = hicl_prototypesᵀ;
 *   eo_mat [D][E] = input_encoder.2.weightᵀ · expert_capability_encoder(expert_embeddings)ᵀ:
 *           the Expert-Oriented head's two linear maps after the SiLU folded into one constant
 *           of the weights (gate.py:362-364);
 *   modal_affinity [E][n_modalities] expert_modal_affinity; expert_bias [E] or NULL.
 * All fp32 except w_proj. heads: the auxiliary heads computed (YVMOE_HEAD_*; the
 * reference skips pruned ones, gate.py:263-276). temperature is the effective one of
 * _safe_temperature (gate.py:297-308), soft_eps = YvNumericalGuard.get_eps(dtype),
 * capacity_loss = 0.005 · Σ relu(usage - limit)² from the usage buffers (gate.py:586-591).
 * Limits: H % 64 == 0, dg_dim % 256 == 0 and <= 32768, 1 <= sparsity_k <= min(64, dg_dim),
 * 1 <= D <= 256.
 */
#define YVMOE_HEAD_HICL 1
#define YVMOE_HEAD_GOT 2
#define YVMOE_HEAD_SOFT 4
#define YVMOE_HEAD_EO 8

typedef struct {
    int32_t num_experts;  /* E */
    int32_t hidden;       /* H */
    int32_t enc_dim;      /* D = expert_embed_dim */
    int32_t dg_dim;       /* hicl_dg_dim = 4H */
    int32_t sparsity_k;   /* min(32, dg_dim) */
    int32_t n_modalities;
    int32_t heads;        /* YVMOE_HEAD_* bits */
    int32_t reserved;
    const void* w_proj;
    const float* dg_bias;
    const float* prototypes_t;
    const float* eo_mat;
    const float* modal_affinity;
    const float* expert_bias;
    float w_hicl, w_got, w_soft, w_eo;
    float soft_temperature;
    float temperature;
    float soft_eps;
    float load_balance_alpha;
    float z_loss_alpha;
    float soft_budget;
    float capacity_loss;
    float reserved_f;
} yvmoe_moegate;

size_t yvmoe_moegate_workspace_bytes(int32_t n_tokens, int32_t act_dtype, const yvmoe_moegate* gate);

/*
 * logits [N][E] fp32: the temperature-scaled logits the gate's softmax and top-k run on;
 * loss [1] fp32: load balance + capacity + z-loss + SoftMoE budget terms of the eval
 * forward (NaN for N = 0, as the reference's means over no tokens). modal_id [N] int32 (one
 * modality per token) or NULL; ids outside [0, n_modalities) add nothing (the module checks
 * them before the call). Route with yvmoe_route on (logits, ld = E) and a yvmoe_router with
 * fixed_shape_mode = 1 and bias = NULL.
 */
int32_t yvmoe_moegate_logits(const void* x, int32_t act_dtype, int32_t n_tokens,
                             const yvmoe_moegate* gate, const int32_t* modal_id, float* logits,
                             float* loss, void* workspace, size_t workspace_bytes, void* stream);

/*
 * The whole eval forward of YvMoEGate (gate.py:310-451 without the PathMoE cache, which is
 * module state): yvmoe_moegate_logits, then the top-k routing of the logits (softmax, top_k,
 * softmax of the k scores, gate.py:393, :414-416) into `routing` (fixed mode: capacity -1),
 * with the expert counts, offsets and permutation of yvmoe_route.
 * workspace: at least yvmoe_moegate_forward_workspace_bytes().
 */
size_t yvmoe_moegate_forward_workspace_bytes(int32_t n_tokens, int32_t act_dtype, int32_t top_k,
                                             const yvmoe_moegate* gate);
int32_t yvmoe_moegate_forward(const void* x, int32_t act_dtype, int32_t n_tokens,
                              const yvmoe_moegate* gate, const int32_t* modal_id, int32_t top_k,
                              float* logits, float* loss, yvmoe_routing* routing,
                              void* workspace, size_t workspace_bytes, void* stream);

/*
 * One YvRMSNorm (model/core/norms.py:178-208): weight [H], bias [H] or NULL, eps.
 */
typedef struct yvmoe_rmsnorm_params {
    const void* weight;
    const void* bias;
    float eps;
    int32_t reserved;
} yvmoe_rmsnorm_params;

/*
 * RMSNorm of the MoE input: n_norms (1 or 2) YvRMSNorms applied in sequence, each as the
 * reference's CUDA path computes it (fused_rms_norm, opss/kernels/fused_rms_norm.py:42,
 * through YvNorms._norm_forward, model/core/norms.py:964-1007): per row rms = sqrt(Σx²/H + eps)
 * in fp32, (x / rms) * weight rounded once to the activation dtype, then + bias (rounded
 * again) when bias is not NULL (norms.py:998-999). Two norms cover the MoE input of
 * YvHybridBlock, norm_mlp(norm_fusion(h)) (model/core/hybrid.py:1359, :1310), in one pass.
 * x, weights, biases and out in the activation dtype, [N][H] row-major, H % 8 == 0; out may
 * alias x.
 */
int32_t yvmoe_rmsnorm(const void* x, int32_t act_dtype, int32_t n_tokens, int32_t hidden,
                      const yvmoe_rmsnorm_params* norms, int32_t n_norms, void* out, void* stream);

/*
 * The whole layer with YvMoEGate as its router, as YvDynamicMoELayer builds it
 * (model/moe/layer.py:754-777, :867-963): yvmoe_moegate_forward, then yvmoe_expert_ffn and
 * yvmoe_combine on that routing. route_logits: NULL to route on this call's logits, or the
 * logits [N][E] of an earlier call to route on instead (the PathMoE stage cache,
 * gate.py:418-431; the loss still comes from this call's logits).
 */
size_t yvmoe_forward_moegate_workspace_bytes(int32_t n_tokens, int32_t act_dtype, int32_t top_k,
                                             const yvmoe_moegate* gate,
                                             const yvmoe_expert_weights* experts);
int32_t yvmoe_forward_moegate(const void* x, int32_t act_dtype, int32_t n_tokens,
                              const yvmoe_moegate* gate, const int32_t* modal_id, int32_t top_k,
                              const float* route_logits, const yvmoe_expert_weights* experts,
                              const float* mix, const void* skip, void* out, void* shared_out,
                              yvmoe_routing* routing, float* logits, float* loss,
                              void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif
#endif /* YVMOE_H */
