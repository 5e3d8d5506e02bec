// YvMoEGate inference forward (model/moe/gate.py:310-451), up to the routing logits and the
// routing loss: every projection of x in one dense GEMM, then one work-group per token builds
// the logits, then one work-group reduces the loss. Routing on the logits is the fixed-mode
// yvmoe_route (softmax, top-k, softmax of the k scores).
//
// Kernels:
//   moegate_proj (dense_gemm_launch): fp32 [N][P] = x · W_projᵀ, W_proj = [dg_proj
//     (hicl_router.py:77); gate; got_cluster_proj; gate_k; gate_v; input_encoder.0; zero
//     rows] — the LDS-tiled MFMA form for batches above 64 rows, the streaming form below.
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
constexpr int kGateCand = 1024;    // most candidates ranked directly (else radix select)
constexpr int kGateGroups = 1024;  // work-groups of the per-token kernel (fixed for a given N)
// Buffer resource word 3 for raw 32-bit buffer loads (data format 32, no swizzle).
constexpr int kBufferFormat = 0x00020000;
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));

struct GateArgs {
    const float* heads;  // row t at heads + t * ld (split z at + z * sstride)
    const float* dg;     // row t at dg + t * ld (split z at + z * sstride)
    int ld;
    int nsplit;          // partial sums of the projection GEMM, summed here in split order
    long long sstride;
    int dgdim;
    int nv;     // DG activations per thread
    int sel_k;  // entries kept
    const float* dg_bias;
    const float* proto_t;
    const float* eo_mat;  // [D][E]
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

// Two reductions in one round: (max of a, sum of b) and (sum of a, sum of b).
template <int NT>
__device__ void block_max_sum(float a, float b, float (*red)[NT / 64], float& ma, float& sb) {
    a = wave_max(a);
    b = wave_sum(b);
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = a;
        red[1][threadIdx.x >> 6] = b;
    }
    __syncthreads();
    ma = red[0][0];
    sb = red[1][0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) {
        ma = fmaxf(ma, red[0][i]);
        sb += red[1][i];
    }
    __syncthreads();
}
template <int NT>
__device__ void block_sum2(float a, float b, float (*red)[NT / 64], float& sa, float& sb) {
    a = wave_sum(a);
    b = wave_sum(b);
    if ((threadIdx.x & 63) == 0) {
        red[0][threadIdx.x >> 6] = a;
        red[1][threadIdx.x >> 6] = b;
    }
    __syncthreads();
    sa = red[0][0];
    sb = red[1][0];
#pragma unroll
    for (int i = 1; i < NT / 64; ++i) {
        sa += red[0][i];
        sb += red[1][i];
    }
    __syncthreads();
}

// Histogram bin b of the radix select lives at b + b / 32: wave 0 reads 32 (or 16)
// consecutive bins per lane without bank conflicts.
__device__ __forceinline__ int hpad(int b) { return b + (b >> 5); }

// Inclusive scans across the 64 lanes of a wave: towards lane 0 (suffix) and from lane 0.
__device__ __forceinline__ unsigned wave_suffix_sum(unsigned v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned t = __shfl_down(v, o);
        if (lane + o < 64) v += t;
    }
    return v;
}
__device__ __forceinline__ unsigned wave_prefix_sum(unsigned v) {
    const int lane = threadIdx.x & 63;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const unsigned t = __shfl_up(v, o);
        if (lane >= o) v += t;
    }
    return v;
}

// Exact radix select over the kGateMaxV keys each thread holds (key(j) == 0: not counted):
// the R-th largest key, in 11/11/10-bit digits. A pass ends early when the bin holding the
// R-th key is counted whole. Result: found = false if fewer than R keys are counted (all of
// them are then taken); else every key > T is taken and, when !whole, the `need` ... of the
// keys equal to T (whole: every key >= T).
struct RadixPick {
    unsigned T, need;
    bool found, whole;
};
template <int NT, class KeyFn>
__device__ RadixPick radix_select(KeyFn key, unsigned R, unsigned* hist, unsigned* ctl) {
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    RadixPick rp{0u, R, true, false};
    unsigned prefix = 0u;
    for (int p = 0; p < 3; ++p) {
        const int sh = p == 0 ? 21 : (p == 1 ? 10 : 0);
        const int nb = p == 2 ? 1024 : 2048;
        const unsigned hmask = p == 0 ? 0u : (~0u << (p == 1 ? 21 : 10));
        for (int b = tid; b < nb + nb / 32; b += NT) hist[b] = 0u;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kGateMaxV; ++j) {
            const unsigned k = key(j);
            if (k != 0u && (k & hmask) == prefix) atomicAdd(&hist[hpad((int)((k >> sh) & (unsigned)(nb - 1)))], 1u);
        }
        __syncthreads();
        if (wave == 0) {
            const int per = nb >> 6;
            unsigned sc = 0u;
            for (int i = 0; i < per; ++i) sc += hist[hpad(lane * per + i)];
            const unsigned S = wave_suffix_sum(sc);  // this lane's bins and all above
            const unsigned total = __shfl(S, 0);
            if (total < rp.need) {
                if (lane == 0) ctl[3] = 1u;
            } else {
                const int L = __ffsll((long long)__ballot(S >= rp.need && S - sc < rp.need)) - 1;
                const unsigned above = __shfl(S - sc, L);
                const int b = L * per + (per - 1 - lane);
                const unsigned h = lane < per ? hist[hpad(b)] : 0u;
                const unsigned P = wave_prefix_sum(h);
                const int c = __ffsll((long long)__ballot(lane < per && above + P >= rp.need)) - 1;
                if (lane == c) {
                    ctl[0] = prefix | ((unsigned)b << sh);
                    ctl[1] = rp.need - (above + P - h);
                    ctl[2] = h;
                    ctl[3] = 0u;
                }
            }
        }
        __syncthreads();
        if (ctl[3]) {  // only in the first pass: fewer than R keys
            rp.found = false;
            break;
        }
        prefix = ctl[0];
        rp.need = ctl[1];
        rp.T = prefix;
        if (ctl[2] == rp.need) {  // the whole bin is taken: every key >= prefix
            rp.whole = true;
            break;
        }
        __syncthreads();  // ctl is rewritten by the next pass
    }
    return rp;
}

// Per token: the DG activations stay in registers (kGateMaxV per thread, 16-byte loads:
// register 4 j4 + c holds index 4 (tid + NT j4) + c). Selection of the sel_k largest:
//   1. a lower bound: the sel_k-th largest of the 64 maxima of 16-lane groups (sel_k groups
//      each hold an element at least that large, so every kept element passes it);
//   2. the elements at or above the bound are appended to a candidate list (typically a few
//      dozen); if more than kGateCand pass, an exact radix select over the float bit
//      patterns (non-negative floats order like their bits) picks the sel_k instead, with a
//      second select over the indices when the sel_k-th value is tied;
//   3. each candidate's rank in (value descending, index ascending) order places it: ranks
//      below sel_k are kept, in that order (ties at the threshold keep the lower indices).
template <int NT, int NS>
__global__ __launch_bounds__(NT) void moegate_token_kernel(GateArgs a) {
    constexpr int Q = NT / 256;  // threads per output of the split dot products
    constexpr int NGRP = NT / 16;
    constexpr int J4 = kGateMaxV / 4;
    static_assert(NT == 1024, "the split dot products assume 4 x 256 threads");
    static_assert(kGateCand <= NT && kGateMaxSel <= NGRP && kGateMaxSel <= 64, "sizes");
    __shared__ unsigned hist[2048 + 64];
    __shared__ float cand_val[kGateCand];
    __shared__ int cand_idx[kGateCand];
    __shared__ float sel_val[kGateMaxSel];
    __shared__ int sel_idx[kGateMaxSel];
    __shared__ float gmax[NGRP];
    __shared__ float s_lk[YVMOE_MAX_EXPERTS];
    __shared__ float s_h[256];
    __shared__ float s_part[Q][256];
    __shared__ float red[2][NT / 64];
    __shared__ unsigned ctl[8];
    __shared__ float s_med, s_tlb;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E, D = a.D, K = a.sel_k;
    const bool is_e = tid < E;
    const int o = tid & 255, q = tid >> 8;  // output and part of the split dot products
    float acc_score = 0.f, acc_z = 0.f, acc_soft = 0.f;

    for (int t = blockIdx.x; t < a.N; t += gridDim.x) {
        const float* hrow = a.heads + (long long)t * a.ld;
        // ---------------------------------------------------------------- HiCL
        float hicl = 0.f;
        if (a.mask & YVMOE_HEAD_HICL) {
            // Buffer loads bounded by the row length: offsets past the row read 0 (on gfx950
            // the range check covers the scalar offset too; rows are whole 1 KB blocks, so a
            // 16-byte load is all in or all out), relu'd to 0 and never kept. The split partial
            // sums are all loaded before any is added (in split order).
            float v[kGateMaxV];
            {
                u32x4 raw[NS][J4];
#pragma unroll
                for (int z = 0; z < NS; ++z) {
                    const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
                        (void*)(a.dg + z * a.sstride + (long long)t * a.ld), 0, a.dgdim * 4, kBufferFormat);
#pragma unroll
                    for (int j4 = 0; j4 < J4; ++j4)
                        raw[z][j4] = __builtin_amdgcn_raw_buffer_load_b128(r, tid * 16, NT * 16 * j4, 0);
                }
                const __amdgpu_buffer_rsrc_t rb =
                    __builtin_amdgcn_make_buffer_rsrc((void*)a.dg_bias, 0, a.dgdim * 4, kBufferFormat);
#pragma unroll
                for (int j4 = 0; j4 < J4; ++j4) {
                    const u32x4 bias = __builtin_amdgcn_raw_buffer_load_b128(rb, tid * 16, NT * 16 * j4, 0);
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        float d = __uint_as_float(raw[0][j4][c]);
#pragma unroll
                        for (int z = 1; z < NS; ++z) d += __uint_as_float(raw[z][j4][c]);
                        d += __uint_as_float(bias[c]);
                        v[4 * j4 + c] = d > 0.f ? d : 0.f;  // +0 for relu'd entries: bit pattern 0
                    }
                }
            }
#define u(j) __float_as_uint(v[j])
            int tid_v = tid;  // opaque per token: keeps the indices from being hoisted
            asm volatile("" : "+v"(tid_v));
#define IDX(j) (4 * (tid_v + NT * ((j) >> 2)) + ((j) & 3))
            // 1. lower bound from the 16-lane group maxima
            float m = 0.f;
#pragma unroll
            for (int j = 0; j < kGateMaxV; ++j) m = fmaxf(m, v[j]);
#pragma unroll
            for (int w = 8; w > 0; w >>= 1) m = fmaxf(m, __shfl_xor(m, w, 16));
            if ((lane & 15) == 0) gmax[tid >> 4] = m;
            __syncthreads();
            if (wave == 0) {
                const float mv = gmax[lane];
                const int mvb = __float_as_int(mv);
                unsigned r = 0u;
#pragma unroll 8
                for (int k = 0; k < NGRP; ++k) {
                    const float g = __int_as_float(__builtin_amdgcn_readlane(mvb, k));
                    r += (g > mv || (g == mv && k < lane)) ? 1u : 0u;
                }
                if (r == (unsigned)(K - 1)) s_tlb = mv;
                if (lane == 0) ctl[5] = 0u;
            }
            __syncthreads();
            const unsigned tlb = __float_as_uint(s_tlb);
            // 2. candidates
#pragma unroll
            for (int j = 0; j < kGateMaxV; ++j) {
                if (u(j) != 0u && u(j) >= tlb) {
                    const unsigned slot = atomicAdd(&ctl[5], 1u);
                    if (slot < (unsigned)kGateCand) {
                        cand_val[slot] = v[j];
                        cand_idx[slot] = IDX(j);
                    }
                }
            }
            __syncthreads();
            int C = (int)ctl[5];
            if (C > kGateCand) {
                __syncthreads();  // every thread has read C: ctl is reused
                const RadixPick rv = radix_select<NT>([&](int j) { return u(j); }, (unsigned)K, hist, ctl);
                unsigned ti = 0u;  // ties at the K-th value: the `need` lowest indices
                if (rv.found && !rv.whole)
                    ti = radix_select<NT>([&](int j) { return u(j) == rv.T ? 32768u - (unsigned)IDX(j) : 0u; },
                                          rv.need, hist, ctl).T;
                if (tid == 0) ctl[5] = 0u;
                __syncthreads();
#pragma unroll
                for (int j = 0; j < kGateMaxV; ++j) {
                    bool take;
                    if (!rv.found) take = u(j) != 0u;
                    else if (rv.whole) take = u(j) >= rv.T;
                    else take = u(j) > rv.T || (u(j) == rv.T && 32768u - (unsigned)IDX(j) >= ti);
                    if (take) {
                        const unsigned slot = atomicAdd(&ctl[5], 1u);
                        if (slot < (unsigned)kGateCand) {
                            cand_val[slot] = v[j];
                            cand_idx[slot] = IDX(j);
                        }
                    }
                }
                __syncthreads();
                C = (int)ctl[5];
            }
#undef u
#undef IDX
            // 3. rank order (value descending, index ascending); ranks below K are kept
            if (C <= 64) {
                if (wave == 0) {
                    const bool in = lane < C;
                    const unsigned mv = in ? __float_as_uint(cand_val[lane]) : 0u;
                    const int mi = in ? cand_idx[lane] : 0;
                    int r = 0;
                    for (int k = 0; k < C; ++k) {
                        const unsigned cv = (unsigned)__builtin_amdgcn_readlane((int)mv, k);
                        const int ci = __builtin_amdgcn_readlane(mi, k);
                        r += (cv > mv || (cv == mv && ci < mi)) ? 1 : 0;
                    }
                    if (in && r < K) {
                        sel_val[r] = __uint_as_float(mv);
                        sel_idx[r] = mi;
                    }
                }
            } else if (tid < C) {
                const unsigned mv = __float_as_uint(cand_val[tid]);
                const int mi = cand_idx[tid];
                int r = 0;
#pragma unroll 8
                for (int k = 0; k < C; ++k) {
                    const unsigned cv = __float_as_uint(cand_val[k]);
                    r += (cv > mv || (cv == mv && cand_idx[k] < mi)) ? 1 : 0;
                }
                if (r < K) {
                    sel_val[r] = __uint_as_float(mv);
                    sel_idx[r] = mi;
                }
            }
            const int nsel = C < K ? C : K;
            __syncthreads();
            if (wave == 0) {  // F.normalize(p=2, eps=1e-12)
                const float x = lane < nsel ? sel_val[lane] : 0.f;
                const float nrm = fmaxf(sqrtf(wave_sum(x * x)), 1e-12f);
                if (lane < nsel) sel_val[lane] = x / nrm;
            }
            __syncthreads();
            float h = 0.f;
            if (o < E) {
                float pv[kGateMaxSel / Q];  // gathers issued together
#pragma unroll
                for (int i = 0; i < kGateMaxSel / Q; ++i) {
                    const int s = q + Q * i;
                    pv[i] = s < nsel ? a.proto_t[(long long)sel_idx[s] * E + o] : 0.f;
                }
#pragma unroll
                for (int i = 0; i < kGateMaxSel / Q; ++i) {
                    const int s = q + Q * i;
                    if (s < nsel) h += sel_val[s] * pv[i];
                }
            }
            s_part[q][o] = h;
            __syncthreads();
            if (is_e) hicl = ((s_part[0][tid] + s_part[1][tid]) + s_part[2][tid]) + s_part[3][tid];
        }
        // ---------------------------------------------------------------- projection heads
        auto hsum = [&](int i) {  // head column i, split partial sums in order
            float sum = hrow[i];
#pragma unroll
            for (int z = 1; z < NS; ++z) sum += hrow[z * a.sstride + i];
            return sum;
        };
        float gate = 0.f, got = 0.f, lk = 0.f, lv = 0.f;
        if (is_e) {
            gate = hsum(tid);
            got = hsum(E + tid);
            lk = hsum(2 * E + tid);
            lv = hsum(3 * E + tid);
            s_lk[tid] = lk;
        }
        if ((a.mask & YVMOE_HEAD_EO) && tid < D) {
            const float hv = hsum(4 * E + tid);
            s_h[tid] = hv / (1.f + expf(-hv));  // SiLU
        }
        __syncthreads();
        // ---------------------------------------------------------------- Expert-Oriented
        // silu(input_encoder.0 x) · M with M = input_encoder.2ᵀ · encoded_expertsᵀ [D][E]
        float eo = 0.f;
        if (a.mask & YVMOE_HEAD_EO) {
            float sum = 0.f;
            if (o < E) {
                for (int d0 = q; d0 < D; d0 += 16 * Q) {  // 16 loads in flight per thread
                    float mv[16];
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int d = d0 + Q * i;
                        mv[i] = d < D ? a.eo_mat[d * E + o] : 0.f;
                    }
#pragma unroll
                    for (int i = 0; i < 16; ++i) {
                        const int d = d0 + Q * i;
                        if (d < D) sum += s_h[d] * mv[i];
                    }
                }
            }
            s_part[q][o] = sum;
            __syncthreads();
            if (is_e) eo = ((s_part[0][tid] + s_part[1][tid]) + s_part[2][tid]) + s_part[3][tid];
        }
        // ---------------------------------------------------------------- SoftMoE, logits, loss
        auto logit = [&](float soft) {
            float l = gate;
            if (a.mask & YVMOE_HEAD_HICL) l = l + a.w_hicl * hicl;
            if (a.mask & YVMOE_HEAD_GOT) l = l + a.w_got * got;
            if (a.mask & YVMOE_HEAD_SOFT) l = l + a.w_soft * soft;
            if (a.mask & YVMOE_HEAD_EO) l = l + a.w_eo * eo;
            if (a.modal_id != nullptr) {
                const int md = a.modal_id[t];
                if (md >= 0 && md < a.nmod) l = l + a.modal[tid * a.nmod + md];
            }
            if (a.ebias != nullptr) l = l + a.ebias[tid];
            l = l / a.temp;
            a.logits[(long long)t * E + tid] = l;
            return l;
        };
        if (E <= 64) {
            // one wavefront holds every expert: wave reductions, no barriers
            if (wave == 0) {
                float soft = 0.f, soft_tot = 0.f;
                if (a.mask & YVMOE_HEAD_SOFT) {
                    // torch.median: the lower middle value (rank, ties by index)
                    const int lkb = __float_as_int(lk);
                    unsigned r = 0u;
                    for (int j = 0; j < E; ++j) {
                        const float x = __int_as_float(__builtin_amdgcn_readlane(lkb, j));
                        r += (x < lk || (x == lk && j < tid)) ? 1u : 0u;
                    }
                    const int ml = __ffsll((long long)__ballot(is_e && r == (unsigned)((E - 1) / 2))) - 1;
                    const float med = __shfl(lk, ml);
                    const float mx = wave_max(is_e ? lv : -INFINITY);
                    const float ex = is_e ? expf(lv - mx) : 0.f;
                    const float se = wave_sum(ex);
                    float sv = is_e ? (1.f / (1.f + expf(-((lk - med) / a.soft_t)))) * (ex / se) : 0.f;
                    sv = sv / fmaxf(wave_sum(sv), a.soft_eps);
                    soft = sv;
                    soft_tot = wave_sum(sv);
                }
                const float l = is_e ? logit(soft) : 0.f;
                const float lm = wave_max(is_e ? l : -INFINITY);
                const float le = is_e ? expf(l - lm) : 0.f;
                const float ls = wave_sum(le);
                if (is_e) acc_score += le / ls;
                const float z = wave_sum(is_e ? l * l : 0.f);
                if (lane == 0) {
                    acc_z += z;
                    acc_soft += soft_tot;
                }
            }
        } else {
            float soft = 0.f, soft_tot = 0.f;
            if (a.mask & YVMOE_HEAD_SOFT) {
                if (is_e) {
                    unsigned r = 0u;
#pragma unroll 8
                    for (int j = 0; j < E; ++j) {
                        const float x = s_lk[j];
                        r += (x < lk || (x == lk && j < tid)) ? 1u : 0u;
                    }
                    if (r == (unsigned)((E - 1) / 2)) s_med = lk;
                }
                const float mx = block_max<NT>(is_e ? lv : -INFINITY, red[0]);
                const float ex = is_e ? expf(lv - mx) : 0.f;
                const float se = block_sum<NT>(ex, red[0]);
                float sv = 0.f;
                if (is_e) sv = (1.f / (1.f + expf(-((lk - s_med) / a.soft_t)))) * (ex / se);
                sv = sv / fmaxf(block_sum<NT>(sv, red[0]), a.soft_eps);
                soft = sv;
            }
            const float l = is_e ? logit(soft) : 0.f;
            float lm, st;
            block_max_sum<NT>(is_e ? l : -INFINITY, soft, red, lm, st);
            soft_tot = st;
            const float le = is_e ? expf(l - lm) : 0.f;
            float ls, z;
            block_sum2<NT>(le, is_e ? l * l : 0.f, red, ls, z);
            if (is_e) acc_score += le / ls;
            if (tid == 0) {
                acc_z += z;
                acc_soft += soft_tot;
            }
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
// 16 waves; wave w sums columns w, w + 16, ... (each lane a fixed stride of groups, then the
// lanes by butterfly), all of its columns' loads in flight together.
constexpr int kLossCols = (YVMOE_MAX_EXPERTS + 2 + 15) / 16;
__global__ __launch_bounds__(1024) void moegate_loss_kernel(const float* __restrict__ part, int G,
                                                            int E, int N, float lb_alpha,
                                                            float z_alpha, float budget,
                                                            float cap_loss, int has_soft,
                                                            float* __restrict__ loss) {
    __shared__ float col[YVMOE_MAX_EXPERTS + 2];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    float s[kLossCols];
#pragma unroll
    for (int i = 0; i < kLossCols; ++i) s[i] = 0.f;
    for (int g = lane; g < G; g += 64) {
#pragma unroll
        for (int i = 0; i < kLossCols; ++i) {
            const int c = wave + 16 * i;
            if (c < E + 2) s[i] += part[(long long)c * G + g];
        }
    }
#pragma unroll
    for (int i = 0; i < kLossCols; ++i) {
        const int c = wave + 16 * i;
        const float v = wave_sum(s[i]);
        if (lane == 0 && c < E + 2) col[c] = v;
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

int moegate_heads_rows(const yvmoe_moegate* g) { return (4 * g->num_experts + g->enc_dim + 255) / 256 * 256; }

int moegate_proj_rows(const yvmoe_moegate* g) {
    return ((g->heads & YVMOE_HEAD_HICL) ? g->dg_dim : 0) + moegate_heads_rows(g);
}

GateWs gate_ws(int N, int act, const yvmoe_moegate* g) {
    GateWs w{};
    const int P = moegate_proj_rows(g);
    const int ks = dense_splits(act, N, P, g->hidden);
    w.groups = N < kGateGroups ? N : kGateGroups;
    size_t o = 0;
    w.proj = o;     o = align_up(o + (size_t)ks * N * P * 4, 256);
    w.loss = o;     o = align_up(o + (size_t)(g->num_experts + 2) * (w.groups > 0 ? w.groups : 1) * 4, 256);
    w.bytes = o;
    return w;
}

int moegate_launch(const void* x, int act, int N, const yvmoe_moegate* g, const int* modal_id,
                   float* logits, float* loss, char* ws, hipStream_t st) {
    const GateWs w = gate_ws(N, act, g);
    const int E = g->num_experts, H = g->hidden;
    const int P = moegate_proj_rows(g);
    const int hoff = (g->heads & YVMOE_HEAD_HICL) ? g->dg_dim : 0;
    float* proj = (float*)(ws + w.proj);
    float* part = (float*)(ws + w.loss);
    if (N > 0) {
        int rc = dense_partials_launch(x, act, N, H, g->w_proj, P, proj, P, st, "moegate_proj");
        if (rc) return rc;
        GateArgs a{};
        a.heads = proj + hoff;
        a.dg = proj;
        a.ld = P;
        a.nsplit = dense_splits(act, N, P, H);
        a.sstride = (long long)N * P;
        a.dgdim = g->dg_dim;
        a.sel_k = g->sparsity_k;
        a.dg_bias = g->dg_bias;
        a.proto_t = g->prototypes_t;
        a.eo_mat = g->eo_mat;
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
        switch (a.nsplit) {
            case 1: moegate_token_kernel<kGateNT, 1><<<w.groups, kGateNT, 0, st>>>(a); break;
            case 2: moegate_token_kernel<kGateNT, 2><<<w.groups, kGateNT, 0, st>>>(a); break;
            default: set_error("moegate: %d partial sums of the projection", a.nsplit); return YVMOE_ERR_SHAPE;
        }
        YV_LAUNCH_CHECK("moegate_token");
    }
    moegate_loss_kernel<<<1, 1024, 0, st>>>(part, w.groups, E, N, g->load_balance_alpha,
                                           g->z_loss_alpha, g->soft_budget, g->capacity_loss,
                                           (g->heads & YVMOE_HEAD_SOFT) ? 1 : 0, loss);
    YV_LAUNCH_CHECK("moegate_loss");
    return YVMOE_OK;
}

}  // namespace yvmoe
