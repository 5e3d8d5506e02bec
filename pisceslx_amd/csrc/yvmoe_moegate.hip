// YvMoEGate inference forward (model/moe/gate.py:310-451), up to the routing logits and the
// routing loss: the projection heads and the DG encoder run on the dense GEMM kernels, then one
// work-group per token builds the logits, then one work-group reduces the loss. Routing on
// the logits is the fixed-mode yvmoe_route (softmax, top-k, softmax of the k scores).
//
// Kernels:
//   moegate_heads / moegate_dg (dense_gemm_launch): fp32 [N][Rh] = x · W_headsᵀ with
//     W_heads = [gate; got_cluster_proj; gate_k; gate_v; input_encoder.0; zero rows], and
//     fp32 [N][dg] = x · dg_projᵀ (hicl_router.py:77).
//   moegate_token_kernel: per token — relu(dg + dg_bias), the sel_k largest kept (radix select
//     on the float bit patterns, ties to the lower index), L2-normalised, dotted with the
//     prototypes (HiCL, gate.py:335-340); the lower median of gate_k, sigmoid, softmax of
//     gate_v, normalisation (SoftMoE, gate.py:351-358); SiLU · input_encoder.2 · encoded
//     expertsᵀ (Expert-Oriented, gate.py:361-366); the weighted sum, modal affinity, expert
//     bias and temperature (gate.py:369-393); per-work-group sums of the softmax scores,
//     logits² and SoftMoE mass for the loss (gate.py:433-444, :556-610).
//   moegate_loss_kernel: the loss from the per-work-group sums, in a fixed order.
#include <math.h>

#include "yvmoe_internal.h"

namespace yvmoe {
namespace {

constexpr int kGateNT = 1024;      // threads of the per-token kernel
constexpr int kGateMaxV = 32;      // DG activations per thread, held in registers (dg <= 32768)
constexpr int kGateMaxSel = 64;    // most DG entries kept per token
constexpr int kGateGroups = 1024;  // work-groups of the per-token kernel (fixed for a given N)
// Buffer resource word 3 for raw 32-bit buffer loads (data format 32, no swizzle).
constexpr int kBufferFormat = 0x00020000;

struct GateArgs {
    const float* heads;
    int ldh;
    const float* dg;
    int dgdim;
    int nv;     // DG activations per thread
    int sel_k;  // entries kept
    const float* dg_bias;
    const float* proto_t;
    const float* enc2_t;
    const float* eenc_t;
    const float* modal;
    int nmod;
    const int* modal_id;
    const float* ebias;
    float w_hicl, w_got, w_soft, w_eo;
    float soft_t, temp, soft_eps;
    int E, D, N, mask;
    float* logits;
    float* part;  // [E + 2][G]
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o));
    return v;
}

// Work-group sum / max; every thread gets the same value (fixed order: lanes by xor
// butterfly, then waves in order).
template <int NT>
__device__ float block_sum(float v, float* red) {
    v = wave_sum(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) s += red[i];
    __syncthreads();
    return s;
}
template <int NT>
__device__ float block_max(float v, float* red) {
    v = wave_max(v);
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
    __syncthreads();
    float s = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) s = fmaxf(s, red[i]);
    __syncthreads();
    return s;
}

// Element j of thread tid is DG index tid + NT * j. For the elements whose bit j is set in
// pm, leaves in cnt[j * W + wave] how many set elements precede lane 0 of (j, wave) in index
// order; an element's rank is that plus the set lanes below it in the same ballot.
template <int NT>
__device__ void ballot_offsets(unsigned long long pm, int nv, unsigned* cnt) {
    constexpr int W = NT / 64;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int j = 0; j < nv; ++j) {
        const unsigned long long m = __ballot((pm >> j) & 1ull);
        if (lane == 0) cnt[j * W + wave] = (unsigned)__popcll(m);
    }
    __syncthreads();
    if (wave == 0) {
        const int n = nv * W;
        const int per = (n + 63) / 64;  // <= 8
        unsigned loc[8];
        unsigned s = 0;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = lane * per + i;
            loc[i] = (i < per && q < n) ? cnt[q] : 0u;
            s += loc[i];
        }
        unsigned P = s;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const unsigned v = __shfl_up(P, o);
            if (lane >= o) P += v;
        }
        unsigned run = P - s;
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const int q = lane * per + i;
            if (i < per && q < n) {
                cnt[q] = run;
                run += loc[i];
            }
        }
    }
    __syncthreads();
}

template <int NT>
__global__ __launch_bounds__(NT) void moegate_token_kernel(GateArgs a) {
    constexpr int W = NT / 64;
    __shared__ unsigned hist[2048];
    __shared__ unsigned cnt[kGateMaxV * W];
    __shared__ float sel_val[kGateMaxSel];
    __shared__ int sel_idx[kGateMaxSel];
    __shared__ float s_lk[YVMOE_MAX_EXPERTS];
    __shared__ float s_h[256];
    __shared__ float s_ie[256];
    __shared__ float red[W];
    __shared__ unsigned ctl[5];
    __shared__ float s_med;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E, D = a.D;
    const bool is_e = tid < E;
    const unsigned long long lt_mask = (1ull << lane) - 1ull;
    float acc_score = 0.f, acc_z = 0.f, acc_soft = 0.f;

    for (int t = blockIdx.x; t < a.N; t += gridDim.x) {
        const float* hrow = a.heads + (long long)t * a.ldh;
        // ---------------------------------------------------------------- HiCL
        float hicl = 0.f;
        if (a.mask & YVMOE_HEAD_HICL) {
            const int nv = a.nv;
            // Buffer loads bounded by the row length: element j sits at a scalar offset from
            // the thread's own, and offsets past the row read 0 (relu'd to 0, never kept).
            const __amdgpu_buffer_rsrc_t rrow = __builtin_amdgcn_make_buffer_rsrc(
                (void*)(a.dg + (long long)t * a.dgdim), 0, a.dgdim * 4, kBufferFormat);
            const __amdgpu_buffer_rsrc_t rbias =
                __builtin_amdgcn_make_buffer_rsrc((void*)a.dg_bias, 0, a.dgdim * 4, kBufferFormat);
            unsigned u[kGateMaxV];
#pragma unroll
            for (int j = 0; j < kGateMaxV; ++j) {
                // the b32 builtin returns the raw bits as an unsigned integer
                const float v =
                    __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rrow, tid * 4, NT * 4 * j, 0)) +
                    __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rbias, tid * 4, NT * 4 * j, 0));
                u[j] = v > 0.f ? __float_as_uint(v) : 0u;
            }
            // The sel_k-th largest relu output as a bit pattern: non-negative floats order
            // like their bits as unsigned integers. Digits of 11, 11 and 10 bits; zeros are
            // never counted (if fewer than sel_k outputs are positive, all positive ones are
            // kept and the zeros add nothing to the norm or the dot products).
            unsigned prefix = 0u, need = (unsigned)a.sel_k, cnt_eq = 0u, npos = 0u;
            bool found = true;
            for (int p = 0; p < 3; ++p) {
                const int sh = p == 0 ? 21 : (p == 1 ? 10 : 0);
                const int nb = p == 2 ? 1024 : 2048;
                const unsigned hmask = p == 0 ? 0u : (~0u << (p == 1 ? 21 : 10));
                for (int b = tid; b < nb; b += NT) hist[b] = 0u;
                __syncthreads();
#pragma unroll
                for (int j = 0; j < kGateMaxV; ++j)
                    if (u[j] != 0u && (u[j] & hmask) == prefix)
                        atomicAdd(&hist[(u[j] >> sh) & (unsigned)(nb - 1)], 1u);
                __syncthreads();
                if (wave == 0) {
                    const int per = nb / 64;
                    unsigned s = 0u;
                    for (int i = 0; i < per; ++i) s += hist[lane * per + i];
                    unsigned S = s;  // count in bins of this lane and all higher lanes
#pragma unroll
                    for (int o = 1; o < 64; o <<= 1) {
                        const unsigned v = __shfl_down(S, o);
                        if (lane + o < 64) S += v;
                    }
                    if (lane == 0) {
                        ctl[3] = S < need ? 1u : 0u;
                        ctl[4] = S;
                    }
                    if (S >= need && S - s < need) {
                        unsigned above = S - s;
                        for (int i = per - 1; i >= 0; --i) {
                            const unsigned h = hist[lane * per + i];
                            if (above + h >= need) {
                                ctl[0] = prefix | ((unsigned)(lane * per + i) << sh);
                                ctl[1] = need - above;
                                ctl[2] = h;
                                break;
                            }
                            above += h;
                        }
                    }
                }
                __syncthreads();
                if (ctl[3]) {  // only possible in the first pass: fewer positives than sel_k
                    found = false;
                    npos = ctl[4];
                    break;
                }
                prefix = ctl[0];
                need = ctl[1];
                cnt_eq = ctl[2];
            }
            const unsigned T = found ? prefix : 0u;
            const int nsel = found ? a.sel_k : (int)npos;
            unsigned long long pm = 0ull;
            if (found && cnt_eq > need) {
                // several elements equal the threshold: keep the `need` lowest indices
                unsigned long long em = 0ull;
#pragma unroll
                for (int j = 0; j < kGateMaxV; ++j) em |= (unsigned long long)(u[j] == T) << j;
                ballot_offsets<NT>(em, nv, cnt);
                for (int j = 0; j < nv; ++j) {
                    const bool e = (em >> j) & 1ull;
                    const unsigned long long m = __ballot(e);
                    if (e && cnt[j * W + wave] + (unsigned)__popcll(m & lt_mask) < need) pm |= 1ull << j;
                }
                __syncthreads();
            }
#pragma unroll
            for (int j = 0; j < kGateMaxV; ++j)
                if (u[j] > T || (found && u[j] == T && cnt_eq == need)) pm |= 1ull << j;
            // compaction of the kept entries in index order
            ballot_offsets<NT>(pm, nv, cnt);
            int tid_v = tid;  // opaque per token: keeps the 32 indices from being hoisted
            asm volatile("" : "+v"(tid_v));
#pragma unroll
            for (int j = 0; j < kGateMaxV; ++j) {  // bits j >= nv are never set
                const bool s = (pm >> j) & 1ull;
                const unsigned long long m = __ballot(s);
                if (s) {
                    const unsigned r = cnt[j * W + wave] + (unsigned)__popcll(m & lt_mask);
                    if (r < (unsigned)kGateMaxSel) {
                        sel_val[r] = __uint_as_float(u[j]);
                        sel_idx[r] = tid_v + NT * j;
                    }
                }
            }
            __syncthreads();
            if (wave == 0) {  // F.normalize(p=2, eps=1e-12)
                const float v = lane < nsel ? sel_val[lane] : 0.f;
                const float nrm = fmaxf(sqrtf(wave_sum(v * v)), 1e-12f);
                if (lane < nsel) sel_val[lane] = v / nrm;
            }
            __syncthreads();
            if (is_e) {
                float h = 0.f;
                for (int i = 0; i < nsel; ++i) h += sel_val[i] * a.proto_t[(long long)sel_idx[i] * E + tid];
                hicl = h;
            }
        }
        // ---------------------------------------------------------------- projection heads
        float gate = 0.f, got = 0.f, lk = 0.f, lv = 0.f;
        if (is_e) {
            gate = hrow[tid];
            got = hrow[E + tid];
            lk = hrow[2 * E + tid];
            lv = hrow[3 * E + tid];
            s_lk[tid] = lk;
        }
        if ((a.mask & YVMOE_HEAD_EO) && tid < D) {
            const float h = hrow[4 * E + tid];
            s_h[tid] = h / (1.f + expf(-h));  // SiLU
        }
        __syncthreads();
        // ---------------------------------------------------------------- SoftMoE
        float soft = 0.f, soft_tot = 0.f;
        if (a.mask & YVMOE_HEAD_SOFT) {
            if (is_e) {  // torch.median: the lower middle value, by rank (ties by index)
                unsigned r = 0u;
                for (int j = 0; j < E; ++j) {
                    const float v = s_lk[j];
                    r += (v < lk || (v == lk && j < tid)) ? 1u : 0u;
                }
                if (r == (unsigned)((E - 1) / 2)) s_med = lk;
            }
            const float mx = block_max<NT>(is_e ? lv : -INFINITY, red);
            const float ex = is_e ? expf(lv - mx) : 0.f;
            const float se = block_sum<NT>(ex, red);
            float sv = 0.f;
            if (is_e) {
                const float sw = 1.f / (1.f + expf(-((lk - s_med) / a.soft_t)));
                sv = sw * (ex / se);
            }
            const float ssum = block_sum<NT>(sv, red);
            sv = sv / fmaxf(ssum, a.soft_eps);
            soft = sv;
            soft_tot = block_sum<NT>(sv, red);
        }
        // ---------------------------------------------------------------- Expert-Oriented
        float eo = 0.f;
        if (a.mask & YVMOE_HEAD_EO) {
            if (tid < D) {
                float s = 0.f;
                for (int d = 0; d < D; ++d) s += s_h[d] * a.enc2_t[d * D + tid];
                s_ie[tid] = s;
            }
            __syncthreads();
            if (is_e) {
                float s = 0.f;
                for (int j = 0; j < D; ++j) s += s_ie[j] * a.eenc_t[j * E + tid];
                eo = s;
            }
        }
        // ---------------------------------------------------------------- logits
        float l = 0.f;
        if (is_e) {
            l = gate;
            if (a.mask & YVMOE_HEAD_HICL) l = l + a.w_hicl * hicl;
            if (a.mask & YVMOE_HEAD_GOT) l = l + a.w_got * got;
            if (a.mask & YVMOE_HEAD_SOFT) l = l + a.w_soft * soft;
            if (a.mask & YVMOE_HEAD_EO) l = l + a.w_eo * eo;
            if (a.modal_id != nullptr) {
                const int m = a.modal_id[t];
                if (m >= 0 && m < a.nmod) l = l + a.modal[tid * a.nmod + m];
            }
            if (a.ebias != nullptr) l = l + a.ebias[tid];
            l = l / a.temp;
            a.logits[(long long)t * E + tid] = l;
        }
        // ---------------------------------------------------------------- loss sums
        const float lm = block_max<NT>(is_e ? l : -INFINITY, red);
        const float le = is_e ? expf(l - lm) : 0.f;
        const float ls = block_sum<NT>(le, red);
        if (is_e) acc_score += le / ls;
        const float z = block_sum<NT>(is_e ? l * l : 0.f, red);
        if (tid == 0) {
            acc_z += z;
            acc_soft += soft_tot;
        }
    }
    const int G = gridDim.x, g = blockIdx.x;
    if (is_e) a.part[(long long)tid * G + g] = acc_score;
    if (tid == 0) {
        a.part[(long long)E * G + g] = acc_z;
        a.part[(long long)(E + 1) * G + g] = acc_soft;
    }
}

// loss = alpha · Σ_e (mean_n score - 1/E)² + capacity term + z_alpha · mean(logits²)
//        + 0.01 · (mean_n Σ_e soft - budget)²   (gate.py:433-444, :556-610)
__global__ __launch_bounds__(256) void moegate_loss_kernel(const float* __restrict__ part, int G,
                                                           int E, int N, float lb_alpha,
                                                           float z_alpha, float budget,
                                                           float cap_loss, int has_soft,
                                                           float* __restrict__ loss) {
    __shared__ float col[YVMOE_MAX_EXPERTS + 2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int c = wave; c < E + 2; c += 4) {
        float s = 0.f;
        for (int g = lane; g < G; g += 64) s += part[(long long)c * G + g];
        s = wave_sum(s);
        if (lane == 0) col[c] = s;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        const float fn = (float)N;
        float lb = 0.f;
        for (int e = 0; e < E; ++e) {
            const float d = col[e] / fn - 1.f / (float)E;
            lb += d * d;
        }
        float total = lb_alpha * lb + cap_loss + z_alpha * (col[E] / ((float)N * (float)E));
        if (has_soft) {
            const float ac = col[E + 1] / fn - budget;
            total += 0.01f * (ac * ac);
        }
        loss[0] = total;
    }
}

}  // namespace

int moegate_heads_rows(const yvmoe_moegate* g) { return pad16(4 * g->num_experts + g->enc_dim); }

GateWs gate_ws(int N, int act, const yvmoe_moegate* g) {
    GateWs w{};
    const int rh = moegate_heads_rows(g);
    const bool hicl = (g->heads & YVMOE_HEAD_HICL) != 0;
    const int ks_h = dense_ksplit(N, rh, g->hidden);
    const int ks_d = dense_ksplit(N, g->dg_dim, g->hidden);
    size_t part = ks_h > 1 ? (size_t)ks_h * N * rh * 4 : 0;
    if (hicl && ks_d > 1) part = part > (size_t)ks_d * N * g->dg_dim * 4 ? part : (size_t)ks_d * N * g->dg_dim * 4;
    w.groups = N < kGateGroups ? N : kGateGroups;
    size_t o = 0;
    w.heads = o;    o = align_up(o + (size_t)N * rh * 4, 256);
    w.dg = o;       o = align_up(o + (hicl ? (size_t)N * g->dg_dim * 4 : 0), 256);
    w.partials = o; o = align_up(o + part, 256);
    w.loss = o;     o = align_up(o + (size_t)(g->num_experts + 2) * (w.groups > 0 ? w.groups : 1) * 4, 256);
    w.bytes = o;
    (void)act;
    return w;
}

int moegate_launch(const void* x, int act, int N, const yvmoe_moegate* g, const int* modal_id,
                   float* logits, float* loss, char* ws, hipStream_t st) {
    const GateWs w = gate_ws(N, act, g);
    const int E = g->num_experts, H = g->hidden;
    const int rh = moegate_heads_rows(g);
    float* heads = (float*)(ws + w.heads);
    float* dg = (float*)(ws + w.dg);
    float* partials = (float*)(ws + w.partials);
    float* part = (float*)(ws + w.loss);
    const bool hicl = (g->heads & YVMOE_HEAD_HICL) != 0;
    if (N > 0) {
        int rc = dense_gemm_launch(x, act, N, H, g->w_heads, rh, heads, rh, partials, st, "moegate_heads");
        if (rc) return rc;
        if (hicl) {
            rc = dense_gemm_launch(x, act, N, H, g->w_dg, g->dg_dim, dg, g->dg_dim, partials, st, "moegate_dg");
            if (rc) return rc;
        }
        GateArgs a{};
        a.heads = heads;
        a.ldh = rh;
        a.dg = dg;
        a.dgdim = g->dg_dim;
        a.sel_k = g->sparsity_k;
        a.dg_bias = g->dg_bias;
        a.proto_t = g->prototypes_t;
        a.enc2_t = g->enc2_t;
        a.eenc_t = g->expert_enc_t;
        a.modal = g->modal_affinity;
        a.nmod = g->n_modalities;
        a.modal_id = modal_id;
        a.ebias = g->expert_bias;
        a.w_hicl = g->w_hicl;
        a.w_got = g->w_got;
        a.w_soft = g->w_soft;
        a.w_eo = g->w_eo;
        a.soft_t = g->soft_temperature;
        a.temp = g->temperature;
        a.soft_eps = g->soft_eps;
        a.E = E;
        a.D = g->enc_dim;
        a.N = N;
        a.mask = g->heads;
        a.logits = logits;
        a.part = part;
        a.nv = ceil_div(g->dg_dim, kGateNT);
        moegate_token_kernel<kGateNT><<<w.groups, kGateNT, 0, st>>>(a);
        YV_LAUNCH_CHECK("moegate_token");
    }
    moegate_loss_kernel<<<1, 256, 0, st>>>(part, w.groups, E, N, g->load_balance_alpha,
                                           g->z_loss_alpha, g->soft_budget, g->capacity_loss,
                                           (g->heads & YVMOE_HEAD_SOFT) ? 1 : 0, loss);
    YV_LAUNCH_CHECK("moegate_loss");
    return YVMOE_OK;
}

}  // namespace yvmoe
