// extern "C" entry points of libyvmoe (declared in include/yvmoe.h): argument checks,
// workspace carving and kernel sequencing. No entry point allocates device memory.
#include <stdarg.h>
#include <stdio.h>

#include <mutex>

#include "yvmoe_internal.h"

namespace yvmoe {

static thread_local char g_err[512] = "";

void set_error(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_err, sizeof g_err, fmt, ap);
    va_end(ap);
}
void clear_error() { g_err[0] = '\0'; }

static int check_router(const yvmoe_router* r, int act) {
    YV_REQUIRE(r != nullptr, YVMOE_ERR_ARG, "router is NULL");
    YV_REQUIRE(r->num_experts >= 1 && r->num_experts <= YVMOE_MAX_EXPERTS, YVMOE_ERR_SHAPE,
               "num_experts=%d outside [1, %d]", r->num_experts, YVMOE_MAX_EXPERTS);
    YV_REQUIRE(r->top_k >= 1 && r->top_k <= r->num_experts && r->top_k <= YVMOE_MAX_TOPK,
               YVMOE_ERR_SHAPE, "top_k=%d outside [1, min(E=%d, %d)]", r->top_k, r->num_experts,
               YVMOE_MAX_TOPK);
    YV_REQUIRE(act == YVMOE_ACT_F32 || act == YVMOE_ACT_BF16, YVMOE_ERR_DTYPE,
               "unknown activation dtype %d", act);
    YV_REQUIRE(r->min_capacity >= 0, YVMOE_ERR_ARG, "min_capacity=%d < 0", r->min_capacity);
    return YVMOE_OK;
}

static int check_experts(const yvmoe_expert_weights* w, int act) {
    YV_REQUIRE(w != nullptr, YVMOE_ERR_ARG, "expert weights are NULL");
    YV_REQUIRE(w->num_routed >= 1 && w->num_routed <= YVMOE_MAX_EXPERTS, YVMOE_ERR_SHAPE,
               "num_routed=%d outside [1, %d]", w->num_routed, YVMOE_MAX_EXPERTS);
    YV_REQUIRE(w->num_shared >= 0 && w->num_shared <= YVMOE_MAX_SHARED, YVMOE_ERR_SHAPE,
               "num_shared=%d outside [0, %d]", w->num_shared, YVMOE_MAX_SHARED);
    YV_REQUIRE(w->hidden > 0 && w->hidden % 64 == 0 && w->ffn > 0 && w->ffn % 64 == 0,
               YVMOE_ERR_SHAPE, "hidden=%d and ffn=%d must be positive multiples of 64",
               w->hidden, w->ffn);
    YV_REQUIRE(w->w_gate && w->w_up && w->w_down, YVMOE_ERR_ARG, "expert weight pointer is NULL");
    switch (w->format) {
        case YVMOE_W_F32:
            YV_REQUIRE(act == YVMOE_ACT_F32, YVMOE_ERR_DTYPE, "fp32 weights need fp32 activations");
            break;
        case YVMOE_W_BF16:
            YV_REQUIRE(act == YVMOE_ACT_BF16, YVMOE_ERR_DTYPE, "bf16 weights need bf16 activations");
            break;
        case YVMOE_W_INT8:
        case YVMOE_W_INT4:
        case YVMOE_W_FP8:
            YV_REQUIRE(act == YVMOE_ACT_BF16, YVMOE_ERR_DTYPE,
                       "quantized weights need bf16 activations");
            YV_REQUIRE(w->s_gate && w->s_up && w->s_down, YVMOE_ERR_ARG,
                       "quantized weights need scales");
            if (w->format != YVMOE_W_INT8)
                YV_REQUIRE(w->hidden % 128 == 0 && w->ffn % 128 == 0, YVMOE_ERR_SHAPE,
                           "int4/fp8 need hidden=%d and ffn=%d multiples of 128", w->hidden, w->ffn);
            break;
        default:
            set_error("unknown weight format %d", w->format);
            return YVMOE_ERR_DTYPE;
    }
    return YVMOE_OK;
}

// With no tokens only counts, offsets and capacity are written (zero-size tensors may
// legitimately carry NULL data pointers).
static int check_routing(const yvmoe_routing* o, int n_tokens) {
    YV_REQUIRE(o != nullptr && o->counts && o->offsets && o->capacity, YVMOE_ERR_ARG,
               "routing output pointer is NULL");
    YV_REQUIRE(n_tokens == 0 || (o->weights && o->indices && o->perm && o->pos), YVMOE_ERR_ARG,
               "routing output pointer is NULL");
    return YVMOE_OK;
}

}  // namespace yvmoe

using namespace yvmoe;

extern "C" {

const char* yvmoe_last_error(void) { return g_err; }

int32_t yvmoe_version(void) { return 1; }

size_t yvmoe_workspace_bytes(int32_t n_tokens, int32_t act_dtype, const yvmoe_router* router,
                             const yvmoe_expert_weights* experts) {
    if (n_tokens < 0 || router == nullptr) return 0;
    const int N = n_tokens, E = router->num_experts, k = router->top_k;
    size_t total = route_ws(N, E, k).bytes;
    if (experts != nullptr)
        total += ffn_ws(N, k, experts->num_routed, experts->num_shared, experts->ffn, act_dtype).bytes;
    total += align_up((size_t)N * router_ld(E, act_dtype) * 4, 256);
    if (experts != nullptr)
        total += y_bytes(N, k, experts->num_shared, experts->hidden, act_dtype);
    total += router_partials_bytes(N, E, act_dtype, router->hidden);
    return total;
}

size_t yvmoe_router_workspace_bytes(int32_t n_tokens, int32_t act_dtype, const yvmoe_router* router) {
    if (n_tokens < 0 || router == nullptr) return 0;
    return router_partials_bytes(n_tokens, router->num_experts, act_dtype, router->hidden);
}

int32_t yvmoe_router_logits(const void* x, int32_t act_dtype, int32_t n_tokens,
                            const yvmoe_router* router, float* logits_out, int32_t ld,
                            void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_router(router, act_dtype);
    if (rc) return rc;
    YV_REQUIRE(n_tokens >= 0, YVMOE_ERR_ARG, "n_tokens=%d < 0", n_tokens);
    if (n_tokens == 0) return YVMOE_OK;
    YV_REQUIRE(x && logits_out && router->w_router, YVMOE_ERR_ARG, "NULL pointer");
    YV_REQUIRE(router->hidden > 0 && router->hidden % 64 == 0, YVMOE_ERR_SHAPE,
               "hidden=%d must be a positive multiple of 64", router->hidden);
    YV_REQUIRE(ld == router_ld(router->num_experts, act_dtype), YVMOE_ERR_SHAPE,
               "ld=%d, expected %d", ld, router_ld(router->num_experts, act_dtype));
    const size_t need = router_partials_bytes(n_tokens, router->num_experts, act_dtype, router->hidden);
    YV_REQUIRE(need == 0 || (workspace != nullptr && workspace_bytes >= need), YVMOE_ERR_WORKSPACE,
               "workspace %zu bytes, need %zu", workspace_bytes, need);
    return router_gemm_launch(x, act_dtype, n_tokens, router, logits_out, ld,
                              need ? (float*)workspace : nullptr, (hipStream_t)stream);
}

int32_t yvmoe_route(const float* logits, int32_t ld, const float* predictor, int32_t n_tokens,
                    const yvmoe_router* router, int32_t capacity_override, yvmoe_routing* out,
                    void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_router(router, YVMOE_ACT_F32);
    if (rc) return rc;
    rc = check_routing(out, n_tokens);
    if (rc) return rc;
    YV_REQUIRE(n_tokens >= 0, YVMOE_ERR_ARG, "n_tokens=%d < 0", n_tokens);
    YV_REQUIRE(n_tokens == 0 || logits, YVMOE_ERR_ARG, "logits are NULL");
    YV_REQUIRE(ld >= router->num_experts, YVMOE_ERR_SHAPE, "ld=%d < E=%d", ld, router->num_experts);
    YV_REQUIRE((long long)n_tokens * router->top_k < (1ll << 31), YVMOE_ERR_SHAPE,
               "N*k overflows int32");
    const size_t need = route_ws(n_tokens, router->num_experts, router->top_k).bytes;
    YV_REQUIRE(workspace != nullptr && workspace_bytes >= need, YVMOE_ERR_WORKSPACE,
               "workspace %zu bytes, need %zu", workspace_bytes, need);
    // predictor columns: ld must be Ep + 64 * terms with terms 1 (fp32) or 3 (bf16)
    const int pterms = (ld - pad16(router->num_experts)) / kPredDim;
    if (predictor != nullptr)
        YV_REQUIRE(pterms == 1 || pterms == 3, YVMOE_ERR_SHAPE,
                   "predictor needs ld = Ep + 64 or Ep + 192, got %d", ld);
    if (!router->fixed_shape_mode && router->dynamic_capacity && capacity_override < 0)
        YV_REQUIRE(predictor && router->b1 && router->w2 && router->b2, YVMOE_ERR_ARG,
                   "dynamic capacity needs the predictor columns and weights");
    return route_launch(logits, ld, predictor, ld, n_tokens, router, capacity_override, out,
                        (char*)workspace, (hipStream_t)stream);
}

int32_t yvmoe_expert_ffn(const void* x, int32_t act_dtype, int32_t n_tokens, int32_t top_k,
                         const yvmoe_expert_weights* experts, const yvmoe_routing* routing,
                         void* y, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_experts(experts, act_dtype);
    if (rc) return rc;
    rc = check_routing(routing, n_tokens);
    if (rc) return rc;
    YV_REQUIRE(n_tokens >= 0, YVMOE_ERR_ARG, "n_tokens=%d < 0", n_tokens);
    YV_REQUIRE(top_k >= 1 && top_k <= YVMOE_MAX_TOPK && top_k <= experts->num_routed,
               YVMOE_ERR_SHAPE, "top_k=%d invalid", top_k);
    if (n_tokens == 0) return YVMOE_OK;
    YV_REQUIRE(x && y, YVMOE_ERR_ARG, "NULL pointer");
    YV_REQUIRE(((uintptr_t)x | (uintptr_t)y | (uintptr_t)workspace) % 16 == 0, YVMOE_ERR_ARG,
               "x, y and workspace must be 16-byte aligned");
    const long long rows = (long long)n_tokens * (top_k + experts->num_shared);
    YV_REQUIRE(rows * experts->hidden < (1ll << 40), YVMOE_ERR_SHAPE, "problem too large");
    const size_t need = route_ws(n_tokens, experts->num_routed, top_k).bytes +
                        ffn_ws(n_tokens, top_k, experts->num_routed, experts->num_shared,
                               experts->ffn, act_dtype).bytes;
    YV_REQUIRE(workspace != nullptr && workspace_bytes >= need, YVMOE_ERR_WORKSPACE,
               "workspace %zu bytes, need %zu", workspace_bytes, need);
    return expert_ffn_launch(x, act_dtype, n_tokens, top_k, experts, routing, y, (char*)workspace,
                             (hipStream_t)stream);
}

size_t yvmoe_dispatch_workspace_bytes(int32_t n_tokens, int32_t act_dtype, int32_t slots_per_token,
                                      const yvmoe_expert_weights* experts) {
    if (n_tokens < 0 || experts == nullptr || slots_per_token < 1 || slots_per_token > YVMOE_MAX_TOPK)
        return 0;
    return dispatch_ws(n_tokens, slots_per_token, experts->num_routed, experts->hidden, experts->ffn,
                       act_dtype).bytes;
}

int32_t yvmoe_dispatch(const void* x, int32_t act_dtype, int32_t n_tokens,
                       const void* routing_weights, int32_t weight_dtype,
                       const int64_t* expert_indices, int32_t slots_per_token,
                       const yvmoe_expert_weights* experts, void* out, void* y_out,
                       int32_t* counts, int32_t* offsets, int32_t* invalid, void* workspace,
                       size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_experts(experts, act_dtype);
    if (rc) return rc;
    const int N = n_tokens, k = slots_per_token, E = experts->num_routed;
    YV_REQUIRE(N >= 0, YVMOE_ERR_ARG, "n_tokens=%d < 0", N);
    YV_REQUIRE(k >= 1 && k <= YVMOE_MAX_TOPK, YVMOE_ERR_SHAPE, "slots_per_token=%d outside [1, %d]",
               k, YVMOE_MAX_TOPK);
    YV_REQUIRE(weight_dtype == YVMOE_ACT_F32 || weight_dtype == YVMOE_ACT_BF16, YVMOE_ERR_DTYPE,
               "routing weights must be fp32 or bf16 (got dtype %d)", weight_dtype);
    YV_REQUIRE((long long)N * k < (1ll << 31) && (long long)N * k * experts->hidden < (1ll << 40),
               YVMOE_ERR_SHAPE, "problem too large");
    const DispatchWs L = dispatch_ws(N, k, E, experts->hidden, experts->ffn, act_dtype);
    YV_REQUIRE(workspace != nullptr && workspace_bytes >= L.bytes, YVMOE_ERR_WORKSPACE,
               "workspace %zu bytes, need %zu", workspace_bytes, L.bytes);
    YV_REQUIRE(N == 0 || (x && out && routing_weights && expert_indices), YVMOE_ERR_ARG,
               "NULL pointer");
    YV_REQUIRE(((uintptr_t)x | (uintptr_t)out | (uintptr_t)y_out | (uintptr_t)workspace) % 16 == 0,
               YVMOE_ERR_ARG, "x, out, y_out and workspace must be 16-byte aligned");
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)workspace;
    int* cnt = counts != nullptr ? counts : (int*)(ws + L.counts);
    int* off = offsets != nullptr ? offsets : (int*)(ws + L.offsets);
    int* misc = (int*)(ws + L.misc);
    int* inv = invalid != nullptr ? invalid : misc + 1;
    int* perm = (int*)(ws + L.perm);
    int* pos = (int*)(ws + L.pos);
    const bool wbf = weight_dtype == YVMOE_ACT_BF16;
    float* w32 = wbf ? (float*)(ws + L.w32) : nullptr;
    rc = dispatch_route_launch(expert_indices, wbf ? (const unsigned short*)routing_weights : nullptr,
                               w32, N, E, k, cnt, off, perm, pos, inv, misc, ws, st);
    if (rc || N == 0) return rc;
    yvmoe_expert_weights routed = *experts;
    routed.num_shared = 0;  // the dispatch runs the routed experts only (fused_moe.py:103-111)
    yvmoe_routing r{};
    r.weights = wbf ? w32 : (float*)routing_weights;
    r.counts = cnt;
    r.offsets = off;
    r.perm = perm;
    r.pos = pos;
    void* y = y_out != nullptr ? y_out : (void*)(ws + L.y);
    rc = expert_ffn_launch(x, act_dtype, N, k, &routed, &r, y, ws, st);
    if (rc) return rc;
    return combine_launch(y, act_dtype, N, experts->hidden, k, 0, &r, nullptr, nullptr, out, nullptr, st);
}

int32_t yvmoe_combine(const void* y, int32_t act_dtype, int32_t n_tokens, int32_t hidden,
                      int32_t top_k, int32_t num_shared, const yvmoe_routing* routing,
                      const float* mix, const void* skip, void* out, void* shared_out,
                      void* stream) {
    clear_error();
    int rc = check_routing(routing, n_tokens);
    if (rc) return rc;
    YV_REQUIRE(act_dtype == YVMOE_ACT_F32 || act_dtype == YVMOE_ACT_BF16, YVMOE_ERR_DTYPE,
               "unknown activation dtype %d", act_dtype);
    YV_REQUIRE(n_tokens >= 0 && hidden > 0 && hidden % 8 == 0, YVMOE_ERR_SHAPE,
               "bad n_tokens=%d / hidden=%d", n_tokens, hidden);
    YV_REQUIRE(top_k >= 1 && top_k <= YVMOE_MAX_TOPK, YVMOE_ERR_SHAPE, "top_k=%d invalid", top_k);
    YV_REQUIRE(num_shared >= 0 && num_shared <= YVMOE_MAX_SHARED, YVMOE_ERR_SHAPE,
               "num_shared=%d invalid", num_shared);
    YV_REQUIRE(num_shared == 0 || mix != nullptr, YVMOE_ERR_ARG, "shared experts need mix weights");
    if (n_tokens == 0) return YVMOE_OK;
    YV_REQUIRE(y && out, YVMOE_ERR_ARG, "NULL pointer");
    return combine_launch(y, act_dtype, n_tokens, hidden, top_k, num_shared, routing, mix, skip,
                          out, shared_out, (hipStream_t)stream);
}

int32_t yvmoe_forward(const void* x, int32_t act_dtype, int32_t n_tokens,
                      const yvmoe_router* router, const yvmoe_expert_weights* experts,
                      const float* mix, const void* skip, void* out, void* shared_out,
                      yvmoe_routing* routing, void* workspace, size_t workspace_bytes,
                      void* stream) {
    clear_error();
    int rc = check_router(router, act_dtype);
    if (rc) return rc;
    rc = check_experts(experts, act_dtype);
    if (rc) return rc;
    rc = check_routing(routing, n_tokens);
    if (rc) return rc;
    YV_REQUIRE(router->num_experts == experts->num_routed && router->hidden == experts->hidden,
               YVMOE_ERR_SHAPE, "router (E=%d, H=%d) and experts (E=%d, H=%d) disagree",
               router->num_experts, router->hidden, experts->num_routed, experts->hidden);
    YV_REQUIRE(n_tokens >= 0, YVMOE_ERR_ARG, "n_tokens=%d < 0", n_tokens);
    const size_t need = yvmoe_workspace_bytes(n_tokens, act_dtype, router, experts);
    YV_REQUIRE(workspace != nullptr && workspace_bytes >= need, YVMOE_ERR_WORKSPACE,
               "workspace %zu bytes, need %zu", workspace_bytes, need);
    YV_REQUIRE(n_tokens == 0 || (x && out), YVMOE_ERR_ARG, "NULL pointer");
    YV_REQUIRE(((uintptr_t)x | (uintptr_t)out | (uintptr_t)workspace) % 16 == 0, YVMOE_ERR_ARG,
               "x, out and workspace must be 16-byte aligned");
    YV_REQUIRE(experts->num_shared == 0 || mix != nullptr, YVMOE_ERR_ARG,
               "shared experts need mix weights");
    hipStream_t st = (hipStream_t)stream;
    const int N = n_tokens, E = router->num_experts, k = router->top_k;
    const int ld = router_ld(E, act_dtype);
    char* ws = (char*)workspace;
    float* logits = (float*)(ws + route_ws(N, E, k).bytes +
                             ffn_ws(N, k, E, experts->num_shared, experts->ffn, act_dtype).bytes);
    void* y = (char*)logits + align_up((size_t)N * ld * 4, 256);
    float* partials = (float*)((char*)y + y_bytes(N, k, experts->num_shared, experts->hidden, act_dtype));
    // The routing's top-k kernels sum the router's split-K partial sums themselves (in split
    // order, as the reduction of yvmoe_router_logits does), so the sums need no launch of their
    // own (above kSmallRouteTok tokens up to kFoldSplits splits: more, read per logit, measured
    // slower than the reduction launch); for small batches the fused routing kernel also builds
    // the expert GEMM tile table.
    const bool small = N > 0 && N <= kSmallRouteTok;
    const int ks = router_ksplit(N, E, act_dtype, router->hidden);
    const bool split = N > 0 && ks > 1 && (small || ks <= kFoldSplits);
    if (N > 0) {
        rc = router_gemm_launch(x, act_dtype, N, router, logits, ld, partials, st, !split);
        if (rc) return rc;
    }
    const float* lsrc = split ? partials : logits;
    const bool need_pred = !router->fixed_shape_mode && router->dynamic_capacity;
    const int S = experts->num_shared;
    TileTable tiles{};
    if (small)
        tiles = ffn_tile_table(N, k, E, S, experts->ffn, act_dtype,
                               ffn_tile_rows(act_dtype, N, k, E, experts->hidden, experts->ffn,
                                             experts->format),
                               ws);
    // the routing kernel builds the tile table unless it has a light part (the FFN builds that)
    const bool tiles_by_route = small && tiles.light == 0;
    rc = route_launch(lsrc, ld, need_pred ? lsrc + pad16(E) : nullptr, ld, N, router, -1, routing,
                      ws, st, split ? ks : 1, (long long)N * ld, tiles_by_route ? &tiles : nullptr);
    if (rc) return rc;
    if (N == 0) return YVMOE_OK;
    rc = expert_ffn_launch(x, act_dtype, N, k, experts, routing, y, ws, st, tiles_by_route);
    if (rc) return rc;
    return combine_launch(y, act_dtype, N, experts->hidden, k, experts->num_shared, routing, mix,
                          skip, out, shared_out, st);
}

}  // extern "C"

namespace yvmoe {

// Scratch of yvmoe_forward_static: one file-scope device array, which every GPU the library
// runs on holds (its own copy at its own address) until the process ends. In host code the
// array's name is a host-side stand-in, not a device address: the kernels get the address
// hipGetSymbolAddress returns for the current device, looked up once per device.
static __device__ __align__(256) unsigned char scratch[YVMOE_STATIC_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kMaxDevices] = {};

static int static_scratch(void** out) {
    int dev = -1;
    hipError_t e = hipGetDevice(&dev);
    YV_REQUIRE(e == hipSuccess && dev >= 0 && dev < kMaxDevices, YVMOE_ERR_LAUNCH,
               "hipGetDevice failed (%s) or device %d beyond %d", hipGetErrorString(e), dev,
               kMaxDevices);
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        YV_REQUIRE(e == hipSuccess && p != nullptr, YVMOE_ERR_LAUNCH,
                   "hipGetSymbolAddress(scratch) on device %d failed: %s", dev, hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return YVMOE_OK;
}

}  // namespace yvmoe

extern "C" {

int32_t yvmoe_forward_static(const void* x, int32_t act_dtype, int32_t n_tokens,
                             const yvmoe_router* router, const yvmoe_expert_weights* experts,
                             const float* mix, const void* skip, void* out, void* shared_out,
                             yvmoe_routing* routing, void* stream) {
    clear_error();
    int rc = check_router(router, act_dtype);
    if (rc) return rc;
    rc = check_experts(experts, act_dtype);
    if (rc) return rc;
    YV_REQUIRE(n_tokens >= 0, YVMOE_ERR_ARG, "n_tokens=%d < 0", n_tokens);
    const size_t need = yvmoe_workspace_bytes(n_tokens, act_dtype, router, experts);
    YV_REQUIRE(need <= (size_t)YVMOE_STATIC_SCRATCH_BYTES, YVMOE_ERR_WORKSPACE,
               "n_tokens=%d needs %zu bytes of scratch, more than the static %zu bytes of "
               "yvmoe_forward_static (use yvmoe_forward with a workspace)",
               n_tokens, need, (size_t)YVMOE_STATIC_SCRATCH_BYTES);
    void* ws = nullptr;
    rc = static_scratch(&ws);
    if (rc) return rc;
    return yvmoe_forward(x, act_dtype, n_tokens, router, experts, mix, skip, out, shared_out,
                         routing, ws, (size_t)YVMOE_STATIC_SCRATCH_BYTES, stream);
}

static int check_moegate(const yvmoe_moegate* g, int act) {
    YV_REQUIRE(g != nullptr, YVMOE_ERR_ARG, "gate is NULL");
    YV_REQUIRE(act == YVMOE_ACT_F32 || act == YVMOE_ACT_BF16, YVMOE_ERR_DTYPE,
               "unknown activation dtype %d", act);
    YV_REQUIRE(g->num_experts >= 1 && g->num_experts <= YVMOE_MAX_EXPERTS, YVMOE_ERR_SHAPE,
               "num_experts=%d outside [1, %d]", g->num_experts, YVMOE_MAX_EXPERTS);
    YV_REQUIRE(g->hidden > 0 && g->hidden % 64 == 0, YVMOE_ERR_SHAPE,
               "hidden=%d must be a positive multiple of 64", g->hidden);
    YV_REQUIRE(g->heads >= 0 && g->heads <= 15, YVMOE_ERR_ARG, "heads=%d", g->heads);
    YV_REQUIRE(g->enc_dim >= 1 && g->enc_dim <= 256, YVMOE_ERR_SHAPE, "enc_dim=%d outside [1, 256]",
               g->enc_dim);
    YV_REQUIRE(g->w_proj != nullptr, YVMOE_ERR_ARG, "w_proj is NULL");
    YV_REQUIRE(g->temperature > 0.f && g->soft_temperature != 0.f, YVMOE_ERR_ARG,
               "temperature=%g soft_temperature=%g", g->temperature, g->soft_temperature);
    YV_REQUIRE(g->n_modalities >= 0, YVMOE_ERR_ARG, "n_modalities=%d", g->n_modalities);
    if (g->heads & YVMOE_HEAD_HICL) {
        YV_REQUIRE(g->dg_dim > 0 && g->dg_dim % 256 == 0 && g->dg_dim <= 32768, YVMOE_ERR_SHAPE,
                   "dg_dim=%d must be a positive multiple of 256 up to 32768", g->dg_dim);
        YV_REQUIRE(g->sparsity_k >= 1 && g->sparsity_k <= 64 && g->sparsity_k <= g->dg_dim,
                   YVMOE_ERR_SHAPE, "sparsity_k=%d outside [1, min(64, dg_dim)]", g->sparsity_k);
        YV_REQUIRE(g->dg_bias && g->prototypes_t, YVMOE_ERR_ARG,
                   "HiCL head needs dg_bias and prototypes_t");
    }
    if (g->heads & YVMOE_HEAD_EO)
        YV_REQUIRE(g->eo_mat != nullptr, YVMOE_ERR_ARG, "expert-oriented head needs eo_mat");
    return YVMOE_OK;
}

size_t yvmoe_moegate_workspace_bytes(int32_t n_tokens, int32_t act_dtype, const yvmoe_moegate* gate) {
    if (n_tokens < 0 || check_moegate(gate, act_dtype) != YVMOE_OK) return 0;
    return gate_ws(n_tokens, act_dtype, gate).bytes;
}

int32_t yvmoe_moegate_logits(const void* x, int32_t act_dtype, int32_t n_tokens,
                             const yvmoe_moegate* gate, const int32_t* modal_id, float* logits,
                             float* loss, void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_moegate(gate, act_dtype);
    if (rc) return rc;
    YV_REQUIRE(n_tokens >= 0, YVMOE_ERR_ARG, "n_tokens=%d < 0", n_tokens);
    YV_REQUIRE(loss != nullptr, YVMOE_ERR_ARG, "loss is NULL");
    YV_REQUIRE(n_tokens == 0 || (x && logits), YVMOE_ERR_ARG, "NULL pointer");
    YV_REQUIRE(modal_id == nullptr || (gate->modal_affinity && gate->n_modalities > 0),
               YVMOE_ERR_ARG, "modal_id needs modal_affinity");
    YV_REQUIRE((long long)n_tokens * (gate->dg_dim > 0 ? gate->dg_dim : 1) < (1ll << 40),
               YVMOE_ERR_SHAPE, "problem too large");
    const size_t need = gate_ws(n_tokens, act_dtype, gate).bytes;
    YV_REQUIRE(workspace != nullptr && workspace_bytes >= need, YVMOE_ERR_WORKSPACE,
               "workspace %zu bytes, need %zu", workspace_bytes, need);
    return moegate_launch(x, act_dtype, n_tokens, gate, modal_id, logits, loss, (char*)workspace,
                          (hipStream_t)stream);
}

size_t yvmoe_moegate_forward_workspace_bytes(int32_t n_tokens, int32_t act_dtype, int32_t top_k,
                                             const yvmoe_moegate* gate) {
    if (n_tokens < 0 || check_moegate(gate, act_dtype) != YVMOE_OK) return 0;
    if (top_k < 1 || top_k > YVMOE_MAX_TOPK || top_k > gate->num_experts) return 0;
    return route_ws(n_tokens, gate->num_experts, top_k).bytes + gate_ws(n_tokens, act_dtype, gate).bytes;
}

int32_t yvmoe_moegate_forward(const void* x, int32_t act_dtype, int32_t n_tokens,
                              const yvmoe_moegate* gate, const int32_t* modal_id, int32_t top_k,
                              float* logits, float* loss, yvmoe_routing* routing,
                              void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_moegate(gate, act_dtype);
    if (rc) return rc;
    rc = check_routing(routing, n_tokens);
    if (rc) return rc;
    const int E = gate->num_experts;
    YV_REQUIRE(top_k >= 1 && top_k <= YVMOE_MAX_TOPK && top_k <= E, YVMOE_ERR_SHAPE,
               "top_k=%d outside [1, min(E=%d, %d)]", top_k, E, YVMOE_MAX_TOPK);
    YV_REQUIRE(n_tokens >= 0, YVMOE_ERR_ARG, "n_tokens=%d < 0", n_tokens);
    YV_REQUIRE(loss != nullptr, YVMOE_ERR_ARG, "loss is NULL");
    YV_REQUIRE(n_tokens == 0 || (x && logits), YVMOE_ERR_ARG, "NULL pointer");
    YV_REQUIRE(modal_id == nullptr || (gate->modal_affinity && gate->n_modalities > 0),
               YVMOE_ERR_ARG, "modal_id needs modal_affinity");
    YV_REQUIRE((long long)n_tokens * top_k < (1ll << 31), YVMOE_ERR_SHAPE, "N*k overflows int32");
    const size_t rbytes = route_ws(n_tokens, E, top_k).bytes;
    const size_t need = rbytes + gate_ws(n_tokens, act_dtype, gate).bytes;
    YV_REQUIRE(workspace != nullptr && workspace_bytes >= need, YVMOE_ERR_WORKSPACE,
               "workspace %zu bytes, need %zu", workspace_bytes, need);
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)workspace;
    // decode sizes: the per-token kernel also runs each token's top-k, and the small-batch
    // routing kernel reduces the loss (two launches fewer)
    const bool small = route_small_fixed(n_tokens);
    const GateTopk tk = route_topk_outputs(n_tokens, E, top_k, routing, ws);
    bool topk_done = false;
    GateLossArgs la{};
    rc = moegate_launch(x, act_dtype, n_tokens, gate, modal_id, logits, loss, ws + rbytes, st,
                        small ? &tk : nullptr, &topk_done, small ? &la : nullptr);
    if (rc) return rc;
    yvmoe_router r{};
    r.num_experts = E;
    r.hidden = gate->hidden;
    r.top_k = top_k;
    r.fixed_shape_mode = 1;
    return route_launch(n_tokens > 0 ? logits : nullptr, E, nullptr, E, n_tokens, &r, -1, routing, ws, st,
                        1, 0, nullptr, topk_done, small ? &la : nullptr);
}

static size_t forward_moegate_bytes(int N, int act, int k, const yvmoe_moegate* g,
                                    const yvmoe_expert_weights* w) {
    const size_t a = gate_ws(N, act, g).bytes;
    const size_t b = ffn_ws(N, k, w->num_routed, w->num_shared, w->ffn, act).bytes +
                     y_bytes(N, k, w->num_shared, w->hidden, act);
    return route_ws(N, g->num_experts, k).bytes + (a > b ? a : b);
}

size_t yvmoe_forward_moegate_workspace_bytes(int32_t n_tokens, int32_t act_dtype, int32_t top_k,
                                             const yvmoe_moegate* gate,
                                             const yvmoe_expert_weights* experts) {
    if (n_tokens < 0 || check_moegate(gate, act_dtype) != YVMOE_OK || experts == nullptr) return 0;
    if (top_k < 1 || top_k > YVMOE_MAX_TOPK || top_k > gate->num_experts) return 0;
    return forward_moegate_bytes(n_tokens, act_dtype, top_k, gate, experts);
}

int32_t yvmoe_forward_moegate(const void* x, int32_t act_dtype, int32_t n_tokens,
                              const yvmoe_moegate* gate, const int32_t* modal_id, int32_t top_k,
                              const float* route_logits, const yvmoe_expert_weights* experts,
                              const float* mix, const void* skip, void* out, void* shared_out,
                              yvmoe_routing* routing, float* logits, float* loss,
                              void* workspace, size_t workspace_bytes, void* stream) {
    clear_error();
    int rc = check_moegate(gate, act_dtype);
    if (rc) return rc;
    rc = check_experts(experts, act_dtype);
    if (rc) return rc;
    rc = check_routing(routing, n_tokens);
    if (rc) return rc;
    const int E = gate->num_experts, k = top_k, S = experts->num_shared;
    YV_REQUIRE(E == experts->num_routed && gate->hidden == experts->hidden, YVMOE_ERR_SHAPE,
               "gate (E=%d, H=%d) and experts (E=%d, H=%d) disagree", E, gate->hidden,
               experts->num_routed, experts->hidden);
    YV_REQUIRE(k >= 1 && k <= YVMOE_MAX_TOPK && k <= E, YVMOE_ERR_SHAPE,
               "top_k=%d outside [1, min(E=%d, %d)]", k, E, YVMOE_MAX_TOPK);
    YV_REQUIRE(n_tokens >= 0, YVMOE_ERR_ARG, "n_tokens=%d < 0", n_tokens);
    YV_REQUIRE(loss != nullptr, YVMOE_ERR_ARG, "loss is NULL");
    YV_REQUIRE(n_tokens == 0 || (x && out && logits), YVMOE_ERR_ARG, "NULL pointer");
    YV_REQUIRE(((uintptr_t)x | (uintptr_t)out | (uintptr_t)workspace) % 16 == 0, YVMOE_ERR_ARG,
               "x, out and workspace must be 16-byte aligned");
    YV_REQUIRE(S == 0 || mix != nullptr, YVMOE_ERR_ARG, "shared experts need mix weights");
    YV_REQUIRE(modal_id == nullptr || (gate->modal_affinity && gate->n_modalities > 0),
               YVMOE_ERR_ARG, "modal_id needs modal_affinity");
    const long long rows = (long long)n_tokens * (k + S);
    YV_REQUIRE(rows * experts->hidden < (1ll << 40) && (long long)n_tokens * k < (1ll << 31),
               YVMOE_ERR_SHAPE, "problem too large");
    const size_t need = forward_moegate_bytes(n_tokens, act_dtype, k, gate, experts);
    YV_REQUIRE(workspace != nullptr && workspace_bytes >= need, YVMOE_ERR_WORKSPACE,
               "workspace %zu bytes, need %zu", workspace_bytes, need);
    hipStream_t st = (hipStream_t)stream;
    char* ws = (char*)workspace;
    const int N = n_tokens;
    const size_t rbytes = route_ws(N, E, k).bytes;
    // the gate's region is reused by the expert FFN once the routing has been computed (the
    // loss reduction, deferred to the routing kernel at decode sizes, reads it first). At decode
    // sizes the per-token kernel also runs each token's top-k, unless the routing comes from a
    // cached PathMoE stage's logits.
    const bool small = route_small_fixed(N);
    const GateTopk tk = route_topk_outputs(N, E, k, routing, ws);
    bool topk_done = false;
    GateLossArgs la{};
    rc = moegate_launch(x, act_dtype, N, gate, modal_id, logits, loss, ws + rbytes, st,
                        (small && route_logits == nullptr) ? &tk : nullptr, &topk_done,
                        small ? &la : nullptr);
    if (rc) return rc;
    yvmoe_router r{};
    r.num_experts = E;
    r.hidden = gate->hidden;
    r.top_k = k;
    r.fixed_shape_mode = 1;
    TileTable tiles{};
    if (small)
        tiles = ffn_tile_table(N, k, E, S, experts->ffn, act_dtype,
                               ffn_tile_rows(act_dtype, N, k, E, experts->hidden, experts->ffn,
                                             experts->format),
                               ws);
    const float* lsrc = route_logits != nullptr ? route_logits : logits;
    const bool tiles_by_route = small && tiles.light == 0;
    rc = route_launch(N > 0 ? lsrc : nullptr, E, nullptr, E, N, &r, -1, routing, ws, st, 1, 0,
                      tiles_by_route ? &tiles : nullptr, topk_done, small ? &la : nullptr);
    if (rc) return rc;
    if (N == 0) return YVMOE_OK;
    void* y = ws + rbytes + ffn_ws(N, k, E, S, experts->ffn, act_dtype).bytes;
    rc = expert_ffn_launch(x, act_dtype, N, k, experts, routing, y, ws, st, tiles_by_route);
    if (rc) return rc;
    return combine_launch(y, act_dtype, N, experts->hidden, k, S, routing, mix, skip, out,
                          shared_out, st);
}

int32_t yvmoe_rmsnorm(const void* x, int32_t act_dtype, int32_t n_tokens, int32_t hidden,
                      const yvmoe_rmsnorm_params* norms, int32_t n_norms, void* out, void* stream) {
    clear_error();
    YV_REQUIRE(act_dtype == YVMOE_ACT_F32 || act_dtype == YVMOE_ACT_BF16, YVMOE_ERR_DTYPE,
               "unknown activation dtype %d", act_dtype);
    YV_REQUIRE(n_tokens >= 0 && hidden > 0 && hidden % 8 == 0, YVMOE_ERR_SHAPE,
               "n_tokens=%d, hidden=%d (a positive multiple of 8)", n_tokens, hidden);
    YV_REQUIRE(norms != nullptr && (n_norms == 1 || n_norms == 2), YVMOE_ERR_ARG,
               "n_norms=%d (1 or 2 norms)", n_norms);
    NormChain nc{};
    for (int n = 0; n < n_norms; ++n) {
        YV_REQUIRE(norms[n].weight != nullptr, YVMOE_ERR_ARG, "norm %d: NULL weight", n);
        YV_REQUIRE(((uintptr_t)norms[n].weight | (uintptr_t)norms[n].bias) % 16 == 0,
                   YVMOE_ERR_ARG, "norm %d: weight and bias must be 16-byte aligned", n);
        YV_REQUIRE(norms[n].eps >= 0.f, YVMOE_ERR_ARG, "norm %d: eps=%g < 0", n, norms[n].eps);
        nc.w[n] = norms[n].weight;
        nc.b[n] = norms[n].bias;
        nc.eps[n] = norms[n].eps;
    }
    if (n_tokens == 0) return YVMOE_OK;
    YV_REQUIRE(x && out, YVMOE_ERR_ARG, "NULL pointer");
    YV_REQUIRE(((uintptr_t)x | (uintptr_t)out) % 16 == 0, YVMOE_ERR_ARG,
               "x and out must be 16-byte aligned");
    return rmsnorm_launch(x, act_dtype, n_tokens, hidden, nc, n_norms, out, (hipStream_t)stream);
}

}  // extern "C"
