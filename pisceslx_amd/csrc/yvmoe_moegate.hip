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

#include <algorithm>

#include "yvmoe_internal.h"
#include "yvmoe_gate_loss.h"
#include "yvmoe_topk.h"

namespace yvmoe {
namespace {

constexpr int kGateMaxSel = 64;    // most DG entries kept per token
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
    int do_topk;  // E <= 64: also the token's top-k (route_topk_small_kernel's outputs)
    GateTopk tk;
};

// Rotation by O lanes inside each row of 16 lanes (DPP row_ror).
template <int O>
__device__ __forceinline__ float ror16(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + O, 0xf, 0xf, false));
}
__device__ __forceinline__ float lane_of(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}
// Wave sum / max, the same value in every lane: rotations by 8, 4, 2, 1 inside each row (each
// step adds two values that the partner lane adds in the other order, so all 16 lanes of a
// row agree bit for bit), then the four row results in row order.
__device__ __forceinline__ float wave_sum(float v) {
    v = v + ror16<8>(v);
    v = v + ror16<4>(v);
    v = v + ror16<2>(v);
    v = v + ror16<1>(v);
    return ((lane_of(v, 0) + lane_of(v, 16)) + lane_of(v, 32)) + lane_of(v, 48);
}
__device__ __forceinline__ float wave_max(float v) {
    v = fmaxf(v, ror16<8>(v));
    v = fmaxf(v, ror16<4>(v));
    v = fmaxf(v, ror16<2>(v));
    v = fmaxf(v, ror16<1>(v));
    return fmaxf(fmaxf(lane_of(v, 0), lane_of(v, 16)), fmaxf(lane_of(v, 32), lane_of(v, 48)));
}
// The m-th smallest (0-based, counted with multiplicity) of the keys of the wavefront's lanes
// that have `valid` set, in every lane: bisection from the top bit, each step one compare, one
// ballot and a population count (scalar) instead of a rank loop over the lanes.
__device__ __forceinline__ unsigned wave_kth_smallest(unsigned key, bool valid, unsigned m) {
    unsigned ans = 0u;
#pragma unroll
    for (int b = 31; b >= 0; --b) {
        const unsigned test = ans | (1u << b);
        if ((unsigned)__popcll(__ballot(valid && key < test)) <= m) ans = test;
    }
    return ans;
}
// fp32 bit patterns mapped to unsigned keys that order like the values (-0 just below +0).
__device__ __forceinline__ unsigned f32_order_key(float x) {
    const unsigned b = __float_as_uint(x);
    return (b >> 31) ? ~b : (b | 0x80000000u);
}
__device__ __forceinline__ float f32_from_order_key(unsigned k) {
    return __uint_as_float((k >> 31) ? (k & 0x7fffffffu) : ~k);
}

// Maximum over each row of 16 lanes.
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, ror16<8>(v));
    v = fmaxf(v, ror16<4>(v));
    v = fmaxf(v, ror16<2>(v));
    return fmaxf(v, ror16<1>(v));
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

// Exact radix select over the JV keys each thread holds (key(j) == 0: not counted):
// the R-th largest key, in 11/11/10-bit digits. A pass ends early when the bin holding the
// R-th key is counted whole. Result: found = false if fewer than R keys are counted (all of
// them are then taken); else every key > T is taken and, when !whole, the `need` ... of the
// keys equal to T (whole: every key >= T).
struct RadixPick {
    unsigned T, need;
    bool found, whole;
};
template <int NT, int JV, class KeyFn>
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
        for (int j = 0; j < JV; ++j) {
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
// register 4 j4 + c holds index 4 (tid + NT j4) + c). Every load that does not depend on the
// selection — the head columns, the expert bias and modal affinity, the expert-oriented
// matrix — is issued with the row loads, so a token waits on global memory twice: the rows,
// then the prototype gathers of the kept entries. Selection of the sel_k largest:
//   1. a lower bound: the sel_k-th largest of the NT / 16 maxima of 16-lane groups (sel_k
//      groups each hold an element at least that large, so every kept element passes it);
//   2. the elements at or above the bound are appended to a candidate list (typically a few
//      dozen); if more than NT pass, an exact radix select over the float bit patterns
//      (non-negative floats order like their bits) picks the sel_k instead, with a second
//      select over the indices when the sel_k-th value is tied;
//   3. each candidate's rank in (value descending, index ascending) order places it: ranks
//      below sel_k are kept, in that order (ties at the threshold keep the lower indices).
// Top-k of one token whose logits (at most 64 experts) are in LDS, by the first 16 lanes of a
// wavefront: route_topk_small_kernel's outputs for the token. Not inlined: its registers would
// otherwise add to the per-token kernel's, which then spills.
__device__ __noinline__ void token_topk(const float* s_rl, int lane, int E, GateTopk tk, int t) {
    int my_id;
    float my_ts, my_w0;
    topk_token<4>([&](int e) { return s_rl[e]; }, nullptr, lane, E, tk.k, my_id, my_ts, my_w0);
    if (lane < tk.k) {
        const size_t sl = (size_t)t * tk.k + lane;
        tk.idx[sl] = (int64_t)my_id;
        tk.topp[sl] = my_ts;
        tk.w0[sl] = my_w0;
    }
}

template <int NT, int NS, int J4>
__global__ __launch_bounds__(NT) void moegate_token_kernel(GateArgs a) {
    constexpr int Q = NT / 256;    // threads per output of the split dot products
    constexpr int NGRP = NT / 16;  // 16-lane groups of the lower bound (sel_k <= NGRP)
    constexpr int CAND = NT;       // most candidates ranked directly (else radix select)
    constexpr int JV = 4 * J4;     // DG activations per thread
    constexpr int EOP = 64 / Q;    // expert-oriented terms prefetched per thread (d < 64)
    static_assert(NT == 512 || NT == 1024, "512 or 1024 threads");
    __shared__ unsigned hist[2048 + 64];
    __shared__ float cand_val[CAND];
    __shared__ int cand_idx[CAND];
    __shared__ float sel_val[kGateMaxSel];
    __shared__ int sel_idx[kGateMaxSel];
    __shared__ float gmax[NGRP];
    __shared__ float s_lk[YVMOE_MAX_EXPERTS];
    __shared__ float s_h[256];
    __shared__ float s_ph[Q][256];  // HiCL dot partial sums
    __shared__ float s_pe[Q][256];  // expert-oriented dot partial sums
    __shared__ float red[2][NT / 64];
    __shared__ unsigned ctl[8];
    __shared__ float s_med, s_tlb;
    __shared__ float s_rl[64];  // the token's logits for its top-k (do_topk)
    __shared__ int s_rank[64];  // candidate ranks (at most 64 candidates)
    __shared__ float s_lv[64];    // gate_v of the token's experts (E <= 64)
    __shared__ float s_soft[65];  // SoftMoE weights of the token's experts, their sum (E <= 64)
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E, D = a.D, K = a.sel_k;
    const bool is_e = tid < E;
    const bool hicl_on = (a.mask & YVMOE_HEAD_HICL) != 0;
    const bool eo_on = (a.mask & YVMOE_HEAD_EO) != 0;
    const int o = tid & 255, q = tid >> 8;  // output and part of the split dot products
    float acc_score = 0.f, acc_z = 0.f, acc_soft = 0.f;

    for (int t = blockIdx.x; t < a.N; t += gridDim.x) {
        const float* hrow = a.heads + (long long)t * a.ld;
        // thread coordinates made opaque per token: keeps the compiler from hoisting every
        // loop-invariant address out of the token loop (and spilling them)
        int tt = tid;
        asm volatile("" : "+v"(tt));
        const int ot = tt & 255, qt = tt >> 8;
        // ---------------------------------------------------------------- loads
        // head columns (split partial sums in order), bias terms, expert-oriented matrix
        float gate = 0.f, got = 0.f, lk = 0.f, lv = 0.f, bias_e = 0.f;
        if (is_e) {
            gate = hrow[tt];
            got = hrow[E + tt];
            lk = hrow[2 * E + tt];
            lv = hrow[3 * E + tt];
#pragma unroll
            for (int z = 1; z < NS; ++z) {
                const float* hz = hrow + z * a.sstride;
                gate += hz[tt];
                got += hz[E + tt];
                lk += hz[2 * E + tt];
                lv += hz[3 * E + tt];
            }
            if (a.ebias != nullptr) bias_e = a.ebias[tt];
        }
        float h1 = 0.f;
        if (eo_on && tid < D) {
            h1 = hrow[4 * E + tt];
#pragma unroll
            for (int z = 1; z < NS; ++z) h1 += hrow[z * a.sstride + 4 * E + tt];
        }
        float em[EOP];  // eo_mat[d][o] for d = q + Q i < 64 (the rest is read at the dot)
        if (eo_on) {
            const float* ecol = a.eo_mat + ot;
#pragma unroll
            for (int i = 0; i < EOP; ++i) {
                const int d = qt + Q * i;
                em[i] = (o < E && d < D) ? ecol[d * E] : 0.f;
            }
        }
        float v[JV];
        if (hicl_on) {
            // Buffer loads bounded by the row length: offsets past the row read 0 (on gfx950
            // the range check covers the scalar offset too; rows are whole 1 KB blocks, so a
            // 16-byte load is all in or all out). Split 0 already holds dg_bias; relu follows
            // the sum of the splits (in split order).
            u32x4 raw[NS][J4];
#pragma unroll
            for (int z = 0; z < NS; ++z) {
                const __amdgpu_buffer_rsrc_t r = __builtin_amdgcn_make_buffer_rsrc(
                    (void*)(a.dg + z * a.sstride + (long long)t * a.ld), 0, a.dgdim * 4, kBufferFormat);
#pragma unroll
                for (int j4 = 0; j4 < J4; ++j4)
                    raw[z][j4] = __builtin_amdgcn_raw_buffer_load_b128(r, tt * 16, NT * 16 * j4, 0);
            }
#pragma unroll
            for (int j4 = 0; j4 < J4; ++j4) {
#pragma unroll
                for (int c = 0; c < 4; ++c) {
                    float d = __uint_as_float(raw[0][j4][c]);
#pragma unroll
                    for (int z = 1; z < NS; ++z) d += __uint_as_float(raw[z][j4][c]);
                    v[4 * j4 + c] = d > 0.f ? d : 0.f;  // +0 for relu'd entries: bit pattern 0
                }
            }
        }
        if (is_e) s_lk[tid] = lk;
        if (is_e && E <= 64) s_lv[tid] = lv;
        if (eo_on && tid < D) s_h[tid] = h1 / (1.f + expf(-h1));  // SiLU
        float modal_e = 0.f;  // affinity of this token's modality (gate.py:369-376)
        if (is_e && a.modal_id != nullptr) {
            const int md = a.modal_id[t];
            if (md >= 0 && md < a.nmod) modal_e = a.modal[tt * a.nmod + md];
        }
        __syncthreads();
        // ---------------------------------------------------------------- Expert-Oriented
        // silu(input_encoder.0 x) · M with M = input_encoder.2ᵀ · encoded_expertsᵀ [D][E]
        if (eo_on) {
            float sum = 0.f;
#pragma unroll
            for (int i = 0; i < EOP; ++i) {
                const int d = q + Q * i;
                if (d < D) sum += s_h[d] * em[i];
            }
            if (o < E)
                for (int d = 64 + q; d < D; d += Q) sum += s_h[d] * a.eo_mat[d * E + ot];
            s_pe[q][o] = sum;
        }
        // ---------------------------------------------------------------- HiCL
        if (hicl_on) {
#define u(j) __float_as_uint(v[j])
#define IDX(j) (4 * (tt + NT * ((j) >> 2)) + ((j) & 3))
            // 1. lower bound from the 16-lane group maxima
            float m = 0.f;
#pragma unroll
            for (int j = 0; j < JV; ++j) m = fmaxf(m, v[j]);
            m = row_max(m);
            if ((lane & 15) == 0) gmax[tid >> 4] = m;
            __syncthreads();
            if (wave == 0) {
                // the sel_k-th largest group maximum = the (NGRP - sel_k)-th smallest (the maxima
                // are non-negative: their bit patterns order like the values)
                const unsigned mv = lane < NGRP ? __float_as_uint(gmax[lane]) : 0u;
                const unsigned th = wave_kth_smallest(mv, lane < NGRP, (unsigned)(NGRP - K));
                if (lane == 0) {
                    s_tlb = __uint_as_float(th);
                    ctl[5] = 0u;
                }
            }
            __syncthreads();
            const unsigned tlb = __float_as_uint(s_tlb);
            if (tid < 64) s_rank[tid] = 0;  // read after the barriers below
            // 2. candidates
#pragma unroll
            for (int j = 0; j < JV; ++j) {
                if (u(j) != 0u && u(j) >= tlb) {
                    const unsigned slot = atomicAdd(&ctl[5], 1u);
                    if (slot < (unsigned)CAND) {
                        cand_val[slot] = v[j];
                        cand_idx[slot] = IDX(j);
                    }
                }
            }
            __syncthreads();
            int C = (int)ctl[5];
            if (C > CAND) {
                __syncthreads();  // every thread has read C: ctl is reused
                const RadixPick rv = radix_select<NT, JV>([&](int j) { return u(j); }, (unsigned)K, hist, ctl);
                unsigned ti = 0u;  // ties at the K-th value: the `need` lowest indices
                if (rv.found && !rv.whole)
                    ti = radix_select<NT, JV>([&](int j) { return u(j) == rv.T ? 32768u - (unsigned)IDX(j) : 0u; },
                                          rv.need, hist, ctl).T;
                if (tid == 0) ctl[5] = 0u;
                __syncthreads();
#pragma unroll
                for (int j = 0; j < JV; ++j) {
                    bool take;
                    if (!rv.found) take = u(j) != 0u;
                    else if (rv.whole) take = u(j) >= rv.T;
                    else take = u(j) > rv.T || (u(j) == rv.T && 32768u - (unsigned)IDX(j) >= ti);
                    if (take) {
                        const unsigned slot = atomicAdd(&ctl[5], 1u);
                        if (slot < (unsigned)CAND) {
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
                // lane i of every wavefront holds candidate i; wavefront w counts the candidates
                // k = w, w + NT / 64, ... that rank above it, and the partial ranks add up in LDS
                const bool in = lane < C;
                const unsigned mv = in ? __float_as_uint(cand_val[lane]) : 0u;
                const int mi = in ? cand_idx[lane] : 0;
                int r = 0;
                for (int k = wave; k < C; k += NT / 64) {
                    const unsigned cv = __float_as_uint(cand_val[k]);
                    const int ci = cand_idx[k];
                    r += (cv > mv || (cv == mv && ci < mi)) ? 1 : 0;
                }
                if (in && r > 0) atomicAdd(&s_rank[lane], r);
                __syncthreads();
                if (wave == 0 && in) {
                    const int rr = s_rank[lane];
                    if (rr < K) {
                        sel_val[rr] = __uint_as_float(mv);
                        sel_idx[rr] = mi;
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
                const float* pcol = a.proto_t + ot;
#pragma unroll
                for (int i = 0; i < kGateMaxSel / Q; ++i) {
                    const int s = q + Q * i;
                    pv[i] = s < nsel ? pcol[(long long)sel_idx[s] * E] : 0.f;
                }
#pragma unroll
                for (int i = 0; i < kGateMaxSel / Q; ++i) {
                    const int s = q + Q * i;
                    if (s < nsel) h += sel_val[s] * pv[i];
                }
            }
            s_ph[q][o] = h;
        }
        // SoftMoE of a gate with at most 64 experts (lane e: expert e), by wavefront 1 beside the
        // HiCL dot products, for wavefront 0's logits after the barrier
        if (E <= 64 && wave == 1 && (a.mask & YVMOE_HEAD_SOFT)) {
            const bool ve = lane < E;
            const float lk1 = ve ? s_lk[lane] : 0.f;
            const float lv1 = ve ? s_lv[lane] : 0.f;
            // torch.median: the lower middle value, the ((E - 1) / 2)-th smallest (equal values
            // have equal bits except +0 and -0, and either as med gives the same sigmoid below)
            const float med = f32_from_order_key(
                wave_kth_smallest(f32_order_key(lk1), ve, (unsigned)((E - 1) / 2)));
            const float mx = wave_max(ve ? lv1 : -INFINITY);
            const float ex = ve ? expf(lv1 - mx) : 0.f;
            const float se = wave_sum(ex);
            float sv = ve ? (1.f / (1.f + expf(-((lk1 - med) / a.soft_t)))) * (ex / se) : 0.f;
            sv = sv / fmaxf(wave_sum(sv), a.soft_eps);
            s_soft[lane] = sv;
            const float tot = wave_sum(sv);
            if (lane == 0) s_soft[64] = tot;
        }
        __syncthreads();
        float hicl = 0.f, eo = 0.f;
        if (is_e) {
            if (hicl_on) {
                hicl = s_ph[0][tid];
#pragma unroll
                for (int i = 1; i < Q; ++i) hicl += s_ph[i][tid];
            }
            if (eo_on) {
                eo = s_pe[0][tid];
#pragma unroll
                for (int i = 1; i < Q; ++i) eo += s_pe[i][tid];
            }
        }
        // ---------------------------------------------------------------- SoftMoE, logits, loss
        auto logit = [&](float soft) {
            float l = gate;
            if (hicl_on) l = l + a.w_hicl * hicl;
            if (a.mask & YVMOE_HEAD_GOT) l = l + a.w_got * got;
            if (a.mask & YVMOE_HEAD_SOFT) l = l + a.w_soft * soft;
            if (eo_on) l = l + a.w_eo * eo;
            if (a.modal_id != nullptr) l = l + modal_e;
            if (a.ebias != nullptr) l = l + bias_e;
            return l / a.temp;
        };
        if (E <= 64) {
            // one wavefront holds every expert: wave reductions, no barriers
            if (wave == 0) {
                float soft = 0.f, soft_tot = 0.f;
                if (a.mask & YVMOE_HEAD_SOFT) {  // from wavefront 1
                    soft = s_soft[tid];
                    soft_tot = s_soft[64];
                }
                const float l = is_e ? logit(soft) : 0.f;
                if (a.do_topk) {
                    // the routing of this token from the logits just written (the bit-exact
                    // top-k of the routing kernels): the wavefront's 64 logits through LDS to its
                    // first 16 lanes, which hold experts l, l + 16, ... as topk_token expects
                    s_rl[tid] = l;
                    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
                    __builtin_amdgcn_wave_barrier();
                    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
                    if (lane < kLanes) token_topk(s_rl, lane, E, a.tk, t);
                    __builtin_amdgcn_wave_barrier();  // s_rl is rewritten by the next token
                }
                // stored after the top-k call, which waits for every outstanding memory access
                if (is_e) a.logits[(long long)t * E + tt] = l;
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
            if (is_e) a.logits[(long long)t * E + tt] = l;
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

// One wavefront per token, for gates of at most 64 experts (lane e holds expert e): no
// work-group barrier inside a token, so a work-group's wavefronts run their tokens
// independently and the per-token latency chain (row loads, selection, prototype gathers)
// overlaps across many tokens. Selection of the sel_k largest DG activations in one pass over
// the row (lane l holds entries 4 (64 j + l) .. + 3, j ascending): a candidate buffer in LDS
// holds, in index order, every entry seen so far that can still be among the sel_k largest,
// and a threshold thr admits only entries above it:
//   - an entry is appended when its relu'd bit pattern exceeds thr (non-negative floats order
//     like their bits; thr starts at 0, so the first entries admitted are the positive ones;
//     the test is one signed integer compare of the raw bits);
//   - when the buffer would overflow it is compacted to exactly the sel_k largest so far (the
//     entries above T, the sel_k-th largest bit pattern found by bisection, and the
//     lowest-index entries equal to T), and thr becomes T: a later entry equal to T ranks
//     after sel_k earlier ones (ties go to the lower index), so it cannot be kept;
//   - after the row, one more compaction leaves the sel_k largest (or all positive entries if
//     fewer), ranked in (value descending, index ascending) order.
constexpr int kWaveTok = 4;     // wavefronts (tokens in flight) per work-group
constexpr int kWaveCand = 512;  // candidate buffer per wavefront (compaction leaves <= 64)
// a compaction leaves at most kGateMaxSel entries, and one row load adds at most 256
static_assert(kWaveCand % 64 == 0 && kWaveCand >= kGateMaxSel + 256, "candidate buffer too small");
// Below this many tokens a wavefront per token cannot stream the rows fast enough (decode, 64
// tokens: 110 us against 71 us for a work-group per token); the work-group form runs instead.
constexpr int kWaveMinTokens = 1024;

template <int NS>
__device__ __forceinline__ float4 dg_load(const GateArgs& a, const float* row, int i4) {
    float4 v = *(const float4*)(row + 4 * i4);
#pragma unroll
    for (int z = 1; z < NS; ++z) {
        const float4 w = *(const float4*)(row + z * a.sstride + 4 * i4);
        v.x += w.x;
        v.y += w.y;
        v.z += w.z;
        v.w += w.w;
    }
    return v;
}
// The same with non-temporal loads (a row that is read once).
template <int NS>
__device__ __forceinline__ float4 dg_load_nt(const GateArgs& a, const float* row, int i4) {
    typedef float f32x4v __attribute__((ext_vector_type(4)));
    f32x4v v = __builtin_nontemporal_load((const f32x4v*)(row + 4 * i4));
#pragma unroll
    for (int z = 1; z < NS; ++z) v += __builtin_nontemporal_load((const f32x4v*)(row + z * a.sstride + 4 * i4));
    return make_float4(v[0], v[1], v[2], v[3]);
}

// Lanes below this one with the flag set in the wavefront mask b.
__device__ __forceinline__ int lanes_below(unsigned long long b) {
    return (int)__builtin_amdgcn_mbcnt_hi((unsigned)(b >> 32), __builtin_amdgcn_mbcnt_lo((unsigned)b, 0u));
}
// Compacts the wavefront's candidate buffer (K <= n <= kWaveCand entries in index order, bit
// patterns of positive floats in cu, none below lo0) to its K largest (ties to the lower
// index), in index order; returns T, the K-th largest bit pattern. The bisection for T runs on
// the entries held in registers and counts with wavefront ballots (one compare per register and
// step; the population counts are scalar work).
__device__ unsigned wave_compact(unsigned* cu, int* ci, int n, int K, unsigned lo0) {
    constexpr int PER = kWaveCand / 64;
    const int lane = threadIdx.x & 63;
    unsigned r[PER];
    unsigned mx = 0u;
#pragma unroll
    for (int m = 0; m < PER; ++m) {
        const int i = 64 * m + lane;
        r[m] = i < n ? cu[i] : 0u;  // 0 never counts: every entry is positive
        mx = max(mx, r[m]);
    }
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) mx = max(mx, (unsigned)__shfl_xor((int)mx, o));
    auto cnt_ge = [&](unsigned x) {
        unsigned c = 0u;
#pragma unroll
        for (int m = 0; m < PER; ++m) c += (unsigned)__popcll(__ballot(r[m] >= x));
        return c;
    };
    unsigned lo = lo0, hi = mx + 1u;  // cnt(lo) = n >= K, cnt(hi) = 0 < K
    while (hi - lo > 1u) {
        const unsigned mid = lo + (hi - lo) / 2u;
        if (cnt_ge(mid) >= (unsigned)K) lo = mid;
        else hi = mid;
    }
    const unsigned T = lo;
    const unsigned need = (unsigned)K - cnt_ge(T + 1u);  // entries equal to T to keep (>= 1)
    // stable compaction, 64 entries at a time (kept entries move to lower or equal positions,
    // and every entry was read into registers above)
    int x[PER];
#pragma unroll
    for (int m = 0; m < PER; ++m) x[m] = 64 * m + lane < n ? ci[64 * m + lane] : 0;
    unsigned ties = 0u;
    int w = 0;
#pragma unroll
    for (int m = 0; m < PER; ++m) {
        const bool tie = r[m] == T;
        const unsigned long long tb = __ballot(tie);
        const unsigned trank = ties + (unsigned)lanes_below(tb);
        const bool keep = r[m] > T || (tie && trank < need);
        const unsigned long long kb = __ballot(keep);
        if (keep) {
            const int pos = w + lanes_below(kb);
            cu[pos] = r[m];
            ci[pos] = x[m];
        }
        ties += (unsigned)__popcll(tb);
        w += __popcll(kb);
    }
    return T;
}

template <int NS>
__global__ __launch_bounds__(64 * kWaveTok) void moegate_wave_kernel(GateArgs a) {
    __shared__ unsigned c_bits[kWaveTok][kWaveCand];
    __shared__ int c_idx[kWaveTok][kWaveCand];
    __shared__ float s_sel[kWaveTok][kGateMaxSel];
    __shared__ int s_sid[kWaveTok][kGateMaxSel];
    __shared__ float s_hh[kWaveTok][256];
    __shared__ float s_part[kWaveTok][66];
    extern __shared__ float s_eo[];  // the Expert-Oriented matrix [D][E], read by every token
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int E = a.E, D = a.D, K = a.sel_k;
    const bool is_e = lane < E;
    const bool hicl_on = (a.mask & YVMOE_HEAD_HICL) != 0;
    const bool eo_on = (a.mask & YVMOE_HEAD_EO) != 0;
    if (eo_on) {
        for (int i = threadIdx.x; i < D * E; i += 64 * kWaveTok) s_eo[i] = a.eo_mat[i];
        __syncthreads();
    }
    const int nj = a.dgdim / 256;  // 16-byte loads per lane per row
    constexpr int BATCH = NS == 1 ? 8 : 4;
    float acc_score = 0.f, acc_z = 0.f, acc_soft = 0.f;

    for (int t = blockIdx.x * kWaveTok + wave; t < a.N; t += gridDim.x * kWaveTok) {
        const float* hrow = a.heads + (long long)t * a.ld;
        // ------------------------------------------------------------ head columns, biases
        float gate = 0.f, got = 0.f, lk = 0.f, lv = 0.f, bias_e = 0.f, modal_e = 0.f;
        if (is_e) {
            gate = hrow[lane];
            got = hrow[E + lane];
            lk = hrow[2 * E + lane];
            lv = hrow[3 * E + lane];
#pragma unroll
            for (int z = 1; z < NS; ++z) {
                const float* hz = hrow + z * a.sstride;
                gate += hz[lane];
                got += hz[E + lane];
                lk += hz[2 * E + lane];
                lv += hz[3 * E + lane];
            }
            if (a.ebias != nullptr) bias_e = a.ebias[lane];
            if (a.modal_id != nullptr) {
                const int md = a.modal_id[t];
                if (md >= 0 && md < a.nmod) modal_e = a.modal[lane * a.nmod + md];
            }
        }
        if (eo_on) {
            for (int d = lane; d < D; d += 64) {
                float h1 = hrow[4 * E + d];
#pragma unroll
                for (int z = 1; z < NS; ++z) h1 += hrow[z * a.sstride + 4 * E + d];
                s_hh[wave][d] = h1 / (1.f + expf(-h1));  // SiLU
            }
        }
        // ------------------------------------------------------------ HiCL
        float hicl = 0.f;
        if (hicl_on) {
            const float* drow = a.dg + (long long)t * a.ld;
            unsigned thr = 0u;
            int n = 0;
            for (int j0 = 0; j0 < nj; j0 += BATCH) {
                float4 v[BATCH];
#pragma unroll
                for (int b = 0; b < BATCH; ++b)
                    if (j0 + b < nj) v[b] = dg_load_nt<NS>(a, drow, (j0 + b) * 64 + lane);
#pragma unroll
                for (int b = 0; b < BATCH; ++b) {
                    if (j0 + b >= nj) continue;
                    // relu'd value above thr <=> the bit pattern, as a signed integer, above thr
                    // (thr < 2^31; negative values and zeros are at most 0 as integers; a NaN
                    // with the sign bit clear counts as the largest, as torch.topk ranks NaN)
                    const int u[4] = {__float_as_int(v[b].x), __float_as_int(v[b].y), __float_as_int(v[b].z),
                                      __float_as_int(v[b].w)};
                    unsigned long long bl[4];
                    int tot = 0;
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        bl[c] = __ballot(u[c] > (int)thr);
                        tot += __popcll(bl[c]);
                    }
                    if (tot == 0) continue;  // wave-uniform
                    if (n + tot > kWaveCand) {
                        thr = wave_compact(c_bits[wave], c_idx[wave], n, K, thr);
                        n = K;
                        tot = 0;
#pragma unroll
                        for (int c = 0; c < 4; ++c) {
                            bl[c] = __ballot(u[c] > (int)thr);
                            tot += __popcll(bl[c]);
                        }
                    }
                    // this lane's entries follow every entry of the lower lanes (index order)
                    int pos = n + lanes_below(bl[0]) + lanes_below(bl[1]) + lanes_below(bl[2]) +
                              lanes_below(bl[3]);
#pragma unroll
                    for (int c = 0; c < 4; ++c) {
                        if (u[c] > (int)thr) {
                            c_bits[wave][pos] = (unsigned)u[c];
                            c_idx[wave][pos] = 4 * ((j0 + b) * 64 + lane) + c;
                            ++pos;
                        }
                    }
                    n += tot;
                }
            }
            if (n > K) {
                wave_compact(c_bits[wave], c_idx[wave], n, K, thr);
                n = K;
            }
            const int C = n;
            // ranks (value descending; the buffer is in index order, so ties by position)
            if (lane < C) {
                const unsigned mv = c_bits[wave][lane];
                int rk = 0;
                for (int k = 0; k < C; ++k) {
                    const unsigned cv = c_bits[wave][k];
                    rk += (cv > mv || (cv == mv && k < lane)) ? 1 : 0;
                }
                s_sel[wave][rk] = __uint_as_float(mv);
                s_sid[wave][rk] = c_idx[wave][lane];
            }
            const int nsel = C;
            // F.normalize(p=2, eps=1e-12)
            const float x = lane < nsel ? s_sel[wave][lane] : 0.f;
            const float nrm = fmaxf(sqrtf(wave_sum(x * x)), 1e-12f);
            if (lane < nsel) s_sel[wave][lane] = x / nrm;
            if (is_e) {
                const float* pcol = a.proto_t + lane;
                for (int s0 = 0; s0 < nsel; s0 += 8) {
                    float pv[8];
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        pv[i] = s0 + i < nsel ? pcol[(long long)s_sid[wave][s0 + i] * E] : 0.f;
#pragma unroll
                    for (int i = 0; i < 8; ++i)
                        if (s0 + i < nsel) hicl += s_sel[wave][s0 + i] * pv[i];
                }
            }
        }
        // ------------------------------------------------------------ Expert-Oriented
        float eo = 0.f;
        if (eo_on && is_e) {
            for (int d = 0; d < D; ++d) eo += s_hh[wave][d] * s_eo[d * E + lane];
        }
        // ------------------------------------------------------------ SoftMoE, logits, loss
        float soft = 0.f, soft_tot = 0.f;
        if (a.mask & YVMOE_HEAD_SOFT) {
            // torch.median: the lower middle value, the ((E - 1) / 2)-th smallest (equal values
            // have equal bits except +0 and -0, and either as med gives the same sigmoid below)
            const float med = f32_from_order_key(
                wave_kth_smallest(f32_order_key(lk), is_e, (unsigned)((E - 1) / 2)));
            const float mx = wave_max(is_e ? lv : -INFINITY);
            const float ex = is_e ? expf(lv - mx) : 0.f;
            const float se = wave_sum(ex);
            float sv = is_e ? (1.f / (1.f + expf(-((lk - med) / a.soft_t)))) * (ex / se) : 0.f;
            sv = sv / fmaxf(wave_sum(sv), a.soft_eps);
            soft = sv;
            soft_tot = wave_sum(sv);
        }
        float l = 0.f;
        if (is_e) {
            l = gate;
            if (hicl_on) l = l + a.w_hicl * hicl;
            if (a.mask & YVMOE_HEAD_GOT) l = l + a.w_got * got;
            if (a.mask & YVMOE_HEAD_SOFT) l = l + a.w_soft * soft;
            if (eo_on) l = l + a.w_eo * eo;
            if (a.modal_id != nullptr) l = l + modal_e;
            if (a.ebias != nullptr) l = l + bias_e;
            l = l / a.temp;
            a.logits[(long long)t * E + lane] = l;
        }
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
    // per-work-group loss sums: the wavefronts' in order
    s_part[wave][lane] = acc_score;
    if (lane == 0) {
        s_part[wave][64] = acc_z;
        s_part[wave][65] = acc_soft;
    }
    __syncthreads();
    const int G = gridDim.x, g = blockIdx.x;
    for (int c = threadIdx.x; c < E + 2; c += 64 * kWaveTok) {
        const int col = c < E ? c : 64 + (c - E);
        float sum = s_part[0][col];
#pragma unroll
        for (int w = 1; w < kWaveTok; ++w) sum += s_part[w][col];
        a.part[(long long)c * G + g] = sum;
    }
}

// The loss from the per-work-group sums (yvmoe_gate_loss.h), in a launch of its own.
__global__ __launch_bounds__(1024) void moegate_loss_kernel(GateLossArgs a) { gate_loss_block(a); }

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
                   float* logits, float* loss, char* ws, hipStream_t st, const GateTopk* topk,
                   bool* topk_done, GateLossArgs* defer_loss) {
    if (topk_done != nullptr) *topk_done = false;
    const GateWs w = gate_ws(N, act, g);
    const int E = g->num_experts, H = g->hidden;
    const int P = moegate_proj_rows(g);
    const int hoff = (g->heads & YVMOE_HEAD_HICL) ? g->dg_dim : 0;
    float* proj = (float*)(ws + w.proj);
    float* part = (float*)(ws + w.loss);
    int groups = w.groups;  // work-groups whose loss sums the loss kernel reads
    if (N > 0) {
        const bool hicl = (g->heads & YVMOE_HEAD_HICL) != 0;
        int rc = dense_partials_launch(x, act, N, H, g->w_proj, P, proj, P, hicl ? g->dg_bias : nullptr,
                                       hicl ? g->dg_dim : 0, st, "moegate_proj");
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
        // 1024 threads: measured faster than two 512-thread work-groups per CU (decode and
        // prefill)
        // 16-byte row loads per thread: 1, 2, 4 or 8 (DG width up to 4K, 8K, 16K, 32K)
        const int j4 = (g->heads & YVMOE_HEAD_HICL) == 0 ? 1 : g->dg_dim <= 4096 ? 1 : g->dg_dim <= 8192 ? 2
                       : g->dg_dim <= 16384 ? 4 : 8;
        a.nv = 4 * j4;
        if (a.nsplit != 1 && a.nsplit != 2) {
            set_error("moegate: %d partial sums of the projection", a.nsplit);
            return YVMOE_ERR_SHAPE;
        }
        if (E <= 64 && N >= kWaveMinTokens && a.nsplit == 1) {
            // a wavefront per token; fewer work-groups than w.groups, so the loss kernel reads
            // this many per-work-group sums
            groups = std::min(ceil_div(N, kWaveTok), kGateGroups);
            const size_t eo_bytes = (g->heads & YVMOE_HEAD_EO) ? (size_t)g->enc_dim * E * 4 : 0;
            // (at these sizes the projection is never split: one partial sum)
            moegate_wave_kernel<1><<<groups, 64 * kWaveTok, eo_bytes, st>>>(a);
            YV_LAUNCH_CHECK("moegate_wave");
        } else {
            if (topk != nullptr && E <= 64) {
                a.do_topk = 1;
                a.tk = *topk;
                if (topk_done != nullptr) *topk_done = true;
            }
#define YV_TOK(NS, J4) moegate_token_kernel<1024, NS, J4><<<w.groups, 1024, 0, st>>>(a)
        switch (j4 * 10 + a.nsplit) {
            case 11: YV_TOK(1, 1); break;
            case 12: YV_TOK(2, 1); break;
            case 21: YV_TOK(1, 2); break;
            case 22: YV_TOK(2, 2); break;
            case 41: YV_TOK(1, 4); break;
            case 42: YV_TOK(2, 4); break;
            case 81: YV_TOK(1, 8); break;
            default: YV_TOK(2, 8); break;
        }
#undef YV_TOK
        YV_LAUNCH_CHECK("moegate_token");
        }
    }
    const GateLossArgs la{part, groups, E, N, g->load_balance_alpha, g->z_loss_alpha, g->soft_budget,
                          g->capacity_loss, (g->heads & YVMOE_HEAD_SOFT) ? 1 : 0, loss};
    if (defer_loss != nullptr) {
        *defer_loss = la;
        return YVMOE_OK;
    }
    moegate_loss_kernel<<<1, 1024, 0, st>>>(la);
    YV_LAUNCH_CHECK("moegate_loss");
    return YVMOE_OK;
}

}  // namespace yvmoe
