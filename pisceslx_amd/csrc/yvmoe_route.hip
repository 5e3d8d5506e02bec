// Routing kernels of the Yv MoE layer for gfx950: softmax, top-k, double softmax,
// dynamic capacity, capacity trim, renormalisation, and the stable expert-sorted
// permutation with prefix-sum offsets.
//
// Reference: YvStableMoEGate.forward model/moe/gate.py:1122-1247 and the sort/bincount/
// cumsum of PiscesLxFusedMoEDispatch.forward opss/infer/fused_moe.py:69-100.
//
// Bit-exactness contract. Given identical fp32 logits, every output here (indices,
// weights, counts, offsets, perm, pos) is bit-identical to the CPU oracle, because both
// follow one arithmetic specification:
//   exp      Cody-Waite reduction (Cephes ln2 split C1 = 0.693359375, C2 = -2.12194440e-4),
//            degree-7 Taylor polynomial in Horner form, exact 2^n scaling, 0 below -86;
//   softmax  max, then 16 partial sums (partial l takes e = l, l+16, ... in order) folded
//            by an xor butterfly 8,4,2,1, then an IEEE divide;
//   top-k    (p desc, expert asc); weights = softmax of the k top p with a sequential sum;
//   capacity tokens of an over-full expert ranked by (p desc, token asc), rank >= cap drop;
//   renorm   (w * kept) / max(sum_j w, 1e-8) with a sequential sum (gate.py:1239-1241).
// This file is compiled with -ffp-contract=off and the pragma below so that no multiply-add
// is fused, and fp32 division is the correctly rounded one.
#pragma clang fp contract(off)

#include "yvmoe_internal.h"
#include "yvmoe_topk.h"
#include "yvmoe_gate_loss.h"

namespace yvmoe {
namespace {

// complexity_predictor of one token by its 16 lanes: sigmoid(w2 . relu(W1 x + b1) + b2)
// (gate.py:930-936); hidden unit c of W1 x is the sum of pred_terms columns q * 64 + c.
// The result is valid on lane 0.
template <typename PredFn>
__device__ __forceinline__ float predictor_token(PredFn predcol, int pred_terms, const float* __restrict__ b1,
                                                 const float* __restrict__ w2, const float* __restrict__ b2,
                                                 int l) {
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kPredDim / kLanes; ++i) {
        const int c = l + kLanes * i;
        float hsum = 0.0f;
        for (int q = 0; q < pred_terms; ++q) hsum = hsum + predcol(q * kPredDim + c);
        hsum = hsum + b1[c];
        hsum = hsum > 0.0f ? hsum : 0.0f;
        acc = acc + w2[c] * hsum;
    }
#define YV_SUMSTEP(O) acc = acc + rot16<O>(acc)
    YV_BFLY16(YV_SUMSTEP);
#undef YV_SUMSTEP
    return 1.0f / (1.0f + expf(-(acc + b2[0])));
}

// One block = 64 tokens, 16 lanes per token, all 64 tokens in one pass (1024 threads).
template <int NV>
__global__ __launch_bounds__(1024) void route_topk_kernel(
    const float* __restrict__ logits, int ld, const float* __restrict__ bias,
    const float* __restrict__ pred, int pred_ld, int pred_terms, const float* __restrict__ b1,
    const float* __restrict__ w2, const float* __restrict__ b2, int N, int E, int k,
    int64_t* __restrict__ idx_out, float* __restrict__ topp, float* __restrict__ w0,
    uint8_t* __restrict__ allowed, int* __restrict__ blockhist, float* __restrict__ blocksum,
    int nsplit, long long sstride) {
    __shared__ int hist[YVMOE_MAX_EXPERTS];
    __shared__ float score[kTokPerBlock];
    const int tid = threadIdx.x;
    const int g = tid / kLanes;
    const int l = tid % kLanes;
    for (int e = tid; e < E; e += blockDim.x) hist[e] = 0;
    if (tid < kTokPerBlock) score[tid] = 0.0f;
    __syncthreads();

    const int tl = g;
    const int t = blockIdx.x * kTokPerBlock + tl;
    if (t < N) {  // uniform across the 16 lanes of a token
        int my_id;
        float my_ts, my_w0;
        // the router GEMM's nsplit (<= kFoldSplits) partial sums (split z at + z * sstride),
        // loaded together and summed in split order
        auto split_sum = [&](const float* q) {
            float t[kFoldSplits];
#pragma unroll
            for (int z = 0; z < kFoldSplits; ++z) t[z] = z < nsplit ? q[z * sstride] : 0.0f;
            float v = t[0];
#pragma unroll
            for (int z = 1; z < kFoldSplits; ++z)
                if (z < nsplit) v = v + t[z];
            return v;
        };
        topk_token<NV>([&](int e) { return split_sum(logits + (size_t)t * ld + e); }, bias, l, E, k, my_id,
                       my_ts, my_w0);
        if (l < k) {
            const size_t s = (size_t)t * k + l;
            idx_out[s] = (int64_t)my_id;
            topp[s] = my_ts;
            w0[s] = my_w0;
            allowed[s] = 1;
            atomicAdd(&hist[my_id], 1);
        }
        if (pred != nullptr) {
            const float sc = predictor_token([&](int c) { return split_sum(pred + (size_t)t * pred_ld + c); },
                                             pred_terms, b1, w2, b2, l);
            if (l == 0) score[tl] = sc;
        }
    }
    __syncthreads();
    for (int e = tid; e < E; e += blockDim.x) blockhist[(size_t)blockIdx.x * E + e] = hist[e];
    if (tid == 0 && pred != nullptr) {
        float s = 0.0f;
        for (int i = 0; i < kTokPerBlock; ++i) s = s + score[i];  // invalid tokens hold 0
        blocksum[blockIdx.x] = s;
    }
}

// cap_mode: 0 = no capacity (fixed_shape_mode), 1 = explicit, 2 = dynamic, 3 = static factor
// blockinv / invalid_out (the dispatch entry; NULL otherwise): per-block counts of slots
// with an expert id outside [0, E), summed into *invalid_out.
__global__ __launch_bounds__(1024) void route_scan_kernel(
    const int* __restrict__ blockhist, int nb, int E, int N, const float* __restrict__ blocksum,
    int cap_mode, int cap_explicit, int min_cap, double cap_factor, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ blockoff, int* __restrict__ cap_out,
    const int* __restrict__ blockinv = nullptr, int* __restrict__ invalid_out = nullptr) {
    __shared__ int part[1024];
    __shared__ int scan[YVMOE_MAX_EXPERTS];
    __shared__ float red[1024];
    __shared__ int s_inv;
    const int tid = threadIdx.x;
    if (tid == 0) s_inv = 0;
    const int C = 1024 / E;  // chunks of blocks per expert (E <= 256 -> C >= 4)
    const int e = tid % E;
    const int c = tid / E;
    const bool active = c < C;
    int b0 = 0, b1 = 0;
    if (active) {
        b0 = (int)((long long)c * nb / C);
        b1 = (int)((long long)(c + 1) * nb / C);
        // eight loads in flight per round trip (a dependent add per load would wait for each)
        int s = 0;
        for (int b = b0; b < b1; b += 8) {
            int v[8];
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = b + j < b1 ? blockhist[(size_t)(b + j) * E + e] : 0;
#pragma unroll
            for (int j = 0; j < 8; ++j) s += v[j];
        }
        part[c * E + e] = s;
    }
    // fixed-order complexity sum: strided per thread, then a fixed tree
    float cs = 0.0f;
    if (cap_mode == 2)
        for (int b = tid; b < nb; b += 1024) cs = cs + blocksum[b];
    red[tid] = cs;
    __syncthreads();
    if (tid < E) {
        int run = 0;
        for (int cc = 0; cc < C; ++cc) {
            const int v = part[cc * E + tid];
            part[cc * E + tid] = run;
            run += v;
        }
        counts[tid] = run;
        scan[tid] = run;
    }
    for (int s = 512; s >= 1; s >>= 1) {
        if (tid < s) red[tid] = red[tid] + red[tid + s];
        __syncthreads();
    }
    // inclusive Hillis-Steele scan of counts over experts
    for (int o = 1; o < E; o <<= 1) {
        int v = 0;
        if (tid < E && tid >= o) v = scan[tid - o];
        __syncthreads();
        if (tid < E) scan[tid] += v;
        __syncthreads();
    }
    if (invalid_out != nullptr) {
        int inv = 0;
        for (int b = tid; b < nb; b += 1024) inv += blockinv[b];
        if (inv) atomicAdd(&s_inv, inv);
    }
    __syncthreads();
    if (tid < E) offsets[tid + 1] = scan[tid];
    if (tid == 0) {
        offsets[0] = 0;
        if (invalid_out != nullptr) *invalid_out = s_inv;
        int cap = -1;
        if (cap_mode == 1) {
            cap = cap_explicit;
        } else if ((cap_mode == 2 || cap_mode == 3) && N == 0) {
            cap = min_cap;  // empty batch: int(0 * cf / E) = 0 -> min_capacity
        } else if (cap_mode == 2 || cap_mode == 3) {
            double cf = cap_factor;
            if (cap_mode == 2) {
                const float avg = red[0] / (float)N;  // complexity_scores.mean() (gate.py:1117)
                cf = 0.5 + 1.5 * (double)avg;
                if (cf > 2.0) cf = 2.0;
                if (cf < 0.5) cf = 0.5;
            }
            cap = (int)((double)N * cf / (double)E);
            if (cap < min_cap) cap = min_cap;
        }
        *cap_out = cap;
    }
    if (active) {
        const int excl = (e == 0 ? 0 : scan[e - 1]);
        int run = excl + part[c * E + e];
        for (int b = b0; b < b1; ++b) {
            const size_t q = (size_t)b * E + e;
            const int v = blockhist[q];
            blockoff[q] = run;
            run += v;
        }
    }
}

// Stable scatter into expert-sorted order: the rank of a slot among same-expert slots of
// its 64-slot chunk comes from 8 wavefront ballots over the expert id bits. A slot whose
// expert id lies outside [0, E) (external indices of the dispatch entry) takes no position:
// pos = -1, and it is left out of every rank and count.
template <typename IdxT>
__global__ __launch_bounds__(256) void route_scatter_kernel(
    const IdxT* __restrict__ idx, int N, int E, int k, const int* __restrict__ blockoff,
    int* __restrict__ perm, int* __restrict__ pos) {
    __shared__ int cnt[YVMOE_MAX_TOPK][YVMOE_MAX_EXPERTS];
    __shared__ unsigned short rk[kTokPerBlock * YVMOE_MAX_TOPK];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const long long base = (long long)blockIdx.x * kTokPerBlock * k;
    const long long total = (long long)N * k;
    const int nslots = (int)((total - base) < (long long)kTokPerBlock * k ? (total - base)
                                                                          : (long long)kTokPerBlock * k);
    const int nchunks = (nslots + 63) / 64;
    auto expert_of = [&](int s, bool& ok) {
        const long long v = (long long)idx[base + s];
        ok = v >= 0 && v < E;
        return ok ? (int)v : 0;
    };
    for (int q = tid; q < nchunks * E; q += 256) cnt[q / E][q % E] = 0;
    __syncthreads();
    for (int c = wave; c < nchunks; c += 4) {
        const int s = c * 64 + lane;
        bool valid = s < nslots;
        int e = 0;
        if (valid) {
            bool ok;
            e = expert_of(s, ok);
            valid = ok;
        }
        unsigned long long mask = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const bool on = (e >> bit) & 1;
            const unsigned long long bb = __ballot(valid && on);
            mask &= on ? bb : ~bb;
        }
        const unsigned long long below = mask & ((1ull << lane) - 1ull);
        if (valid) {
            rk[s] = (unsigned short)__popcll(below);
            if (below == 0ull) cnt[c][e] = __popcll(mask);
        }
    }
    __syncthreads();
    for (int e = tid; e < E; e += 256) {
        int run = 0;
        for (int c = 0; c < nchunks; ++c) {
            const int v = cnt[c][e];
            cnt[c][e] = run;
            run += v;
        }
    }
    __syncthreads();
    for (int s = tid; s < nslots; s += 256) {
        bool ok;
        const int e = expert_of(s, ok);
        const long long slot = base + s;
        if (!ok) {
            pos[slot] = -1;
            continue;
        }
        const int p = blockoff[(size_t)blockIdx.x * E + e] + cnt[s / 64][e] + rk[s];
        perm[p] = (int)slot;
        pos[slot] = p;
    }
}

// Capacity trim of one expert: LDS radix select of the cap-th largest p (4 passes of 8
// bits on the fp32 bit pattern, which orders like the value for p >= 0), then keep
// p > T and the first (cap - #{p > T}) slots with p == T in token order (gate.py:1228-1236).
// The first kTrimKeys x 256 slots' keys are gathered once (perm, then p) into registers, so
// the five passes over them read no memory; slots past those are gathered on every pass.
constexpr int kTrimKeys = 16;
__global__ __launch_bounds__(256) void capacity_trim_kernel(
    const int* __restrict__ counts, const int* __restrict__ offsets, const int* __restrict__ cap_ptr,
    const int* __restrict__ perm, const float* __restrict__ topp, uint8_t* __restrict__ allowed) {
    __shared__ unsigned hist[256];
    __shared__ unsigned s_prefix;
    __shared__ int s_rem;
    __shared__ int wave_tot[4];
    const int e = blockIdx.x;
    const int n = counts[e];
    const int cap = *cap_ptr;
    if (cap < 0 || n <= cap) return;
    const int off = offsets[e];
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    if (cap == 0) {  // every slot of the expert is surplus (gate.py:1231-1236 with cap 0)
        for (int i = tid; i < n; i += 256) allowed[perm[off + i]] = 0;
        return;
    }
    // slot i = tid + 256 j of the expert: j < kTrimKeys cached (slot index and key)
    int cs[kTrimKeys];
    unsigned ck[kTrimKeys];
#pragma unroll
    for (int j = 0; j < kTrimKeys; ++j) {
        const int i = tid + 256 * j;
        cs[j] = i < n ? perm[off + i] : -1;
    }
#pragma unroll
    for (int j = 0; j < kTrimKeys; ++j) ck[j] = cs[j] >= 0 ? __float_as_uint(topp[cs[j]]) : 0u;
    unsigned prefix = 0u, pmask = 0u;
    int rem = cap;
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[tid] = 0u;
        __syncthreads();
#pragma unroll
        for (int j = 0; j < kTrimKeys; ++j) {
            if (cs[j] >= 0 && (ck[j] & pmask) == prefix) atomicAdd(&hist[(ck[j] >> shift) & 255u], 1u);
        }
        for (int i = tid + 256 * kTrimKeys; i < n; i += 256) {
            const unsigned key = __float_as_uint(topp[perm[off + i]]);
            if ((key & pmask) == prefix) atomicAdd(&hist[(key >> shift) & 255u], 1u);
        }
        __syncthreads();
        if (wave == 0) {
            // lane l owns bins 255-4l .. 252-4l (descending)
            unsigned h[4];
            unsigned loc = 0u;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                h[i] = hist[255 - (4 * lane + i)];
                loc += h[i];
            }
            unsigned incl = loc;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const unsigned v = __shfl_up(incl, o, 64);
                if (lane >= o) incl += v;
            }
            unsigned cum = incl - loc;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                if (cum < (unsigned)rem && cum + h[i] >= (unsigned)rem) {
                    s_prefix = prefix | ((unsigned)(255 - (4 * lane + i)) << shift);
                    s_rem = rem - (int)cum;
                }
                cum += h[i];
            }
        }
        __syncthreads();
        prefix = s_prefix;
        rem = s_rem;
        pmask |= 255u << shift;
        __syncthreads();
    }
    const unsigned T = prefix;
    int running = 0;
    for (int b = 0, j = 0; b < n; b += 256, ++j) {
        const int i = b + tid;
        const bool valid = i < n;
        int slot = -1;
        unsigned key = 0u;
        if (j < kTrimKeys) {
            // registers cs / ck by a uniform index: a select chain, no scratch
#pragma unroll
            for (int jj = 0; jj < kTrimKeys; ++jj) {
                if (jj == j) {
                    slot = cs[jj];
                    key = ck[jj];
                }
            }
        } else if (valid) {
            slot = perm[off + i];
            key = __float_as_uint(topp[slot]);
        }
        const bool iseq = valid && key == T;
        const unsigned long long m = __ballot(iseq);
        const int rw = __popcll(m & ((1ull << lane) - 1ull));
        if (lane == 0) wave_tot[wave] = __popcll(m);
        __syncthreads();
        int before = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < 4; ++w) {
            if (w < wave) before += wave_tot[w];
            tot += wave_tot[w];
        }
        const bool keep = key > T || (iseq && running + before + rw < rem);
        if (valid && !keep) allowed[slot] = 0;
        running += tot;
        __syncthreads();
    }
}

__global__ __launch_bounds__(256) void renorm_kernel(const float* __restrict__ w0,
                                                     const uint8_t* __restrict__ allowed, int N,
                                                     int k, float* __restrict__ w) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= N) return;
    float tmp[YVMOE_MAX_TOPK];
    float tot = 0.0f;
    for (int j = 0; j < k; ++j) {
        const size_t s = (size_t)t * k + j;
        tmp[j] = w0[s] * (allowed[s] ? 1.0f : 0.0f);
        tot = tot + tmp[j];
    }
    const float den = tot > 1e-8f ? tot : 1e-8f;
    const float keep = tot > 0.0f ? 1.0f : 0.0f;
    for (int j = 0; j < k; ++j) w[(size_t)t * k + j] = (tmp[j] * keep) / den;
}

// ------------------------------------------------------------------ small batches
// Routing of a batch of up to kSmallRouteTok tokens (decode) in two launches.
//
// route_topk_small_kernel: one token per work-group of 256 threads. The token's logits and
// predictor columns are first summed over the router GEMM's K splits, in split order (the
// order of reduce_splits_kernel), into LDS with all loads in flight; then the per-token
// top-k and predictor run from LDS (topk_token, predictor_token: the same code as the
// multi-block path).
//
// route_small_kernel: one work-group of 1024 threads for the rest: histogram, scan and
// capacity (the fixed-order complexity sums of the multi-block path: per 64-token block in
// token order, then the same 1024-wide tree), the stable scatter, the capacity trim, the
// renormalisation, and the expert GEMM tile table. The trim ranks the slots of an over-full
// expert by (p desc, token asc) directly, which keeps the same set as the radix select of
// capacity_trim_kernel (p > T, then the first ties in token order).
constexpr int kSmallSlots = kSmallRouteTok * YVMOE_MAX_TOPK;
constexpr int kSmallChunks = kSmallSlots / 64;
constexpr int kMaxPredTerms = 3;  // predictor columns per hidden unit held in LDS

// One token per work-group of 256 threads: each thread reduces about one column over the K
// splits (all split loads of a column in flight together), then the token's 16 lanes run
// the top-k and the predictor from LDS.
template <int NV>
__global__ __launch_bounds__(256) void route_topk_small_kernel(
    const float* __restrict__ logits, const float* __restrict__ pred, int ld, int ksplit,
    long long split_stride, int pred_terms, const float* __restrict__ bias, const float* __restrict__ b1,
    const float* __restrict__ w2, const float* __restrict__ b2, int N, int E, int k,
    int64_t* __restrict__ idx_out, float* __restrict__ topp, float* __restrict__ w0,
    float* __restrict__ score) {
    __shared__ float s_lg[16 * NV];
    __shared__ float s_pr[kMaxPredTerms * kPredDim];
    __shared__ float s_bias[16 * NV];
    __shared__ float s_b1[kPredDim], s_w2[kPredDim], s_b2[1];
    const int tid = threadIdx.x;
    const int t = blockIdx.x;
    const int npc = (pred != nullptr) ? pred_terms * kPredDim : 0;
    // the bias and predictor constants into LDS, loaded alongside the partial sums below
    // (the top-k and predictor then wait on one round of global loads, not two)
    if (bias != nullptr && tid < E) s_bias[tid] = bias[tid];
    if (pred != nullptr) {
        if (tid < kPredDim) {
            s_b1[tid] = b1[tid];
            s_w2[tid] = w2[tid];
        }
        if (tid == kPredDim) s_b2[0] = b2[0];
    }
    for (int c = tid; c < E + npc; c += 256) {
        const float* base = (c < E) ? logits + (size_t)t * ld + c : pred + (size_t)t * ld + (c - E);
        // unconditional loads (split index clamped): no branch, so all are in flight together
        float part[16];
#pragma unroll
        for (int z = 0; z < 16; ++z) part[z] = base[(size_t)min(z, ksplit - 1) * split_stride];
        float v = part[0];
#pragma unroll
        for (int z = 1; z < 16; ++z) v = (z < ksplit) ? v + part[z] : v;
        for (int z = 16; z < ksplit; ++z) v = v + base[(size_t)z * split_stride];
        if (c < E) s_lg[c] = v;
        else s_pr[c - E] = v;
    }
    __syncthreads();
    // no barrier follows: the top-k runs on wavefront 0's first 16 lanes and, at the same time,
    // the predictor on wavefront 1's first 16 lanes (both read only LDS)
    if (tid < kLanes) {
        const int l = tid;
        int my_id;
        float my_ts, my_w0;
        topk_token<NV>([&](int e) { return s_lg[e]; }, bias != nullptr ? s_bias : nullptr, l, E, k, my_id,
                       my_ts, my_w0);
        if (l < k) {
            const size_t s = (size_t)t * k + l;
            idx_out[s] = (int64_t)my_id;
            topp[s] = my_ts;
            w0[s] = my_w0;
        }
    } else if (pred != nullptr && tid >= 64 && tid < 64 + kLanes) {
        const int l = tid - 64;
        const float sv = predictor_token([&](int c) { return s_pr[c]; }, pred_terms, s_b1, s_w2, s_b2, l);
        if (l == 0) score[t] = sv;
    }
}

struct SmallRouteArgs {
    int N, E, k;
    int cap_mode, cap_explicit, min_cap;
    double cap_factor;
    const int64_t* indices;
    const float* topp;
    const float* w0;
    const float* score;
    float* weights;
    int* counts;
    int* offsets;
    int* perm;
    int* pos;
    int* cap_out;
    TileTable tiles;  // tiles.seg == nullptr: no tile table
    int has_loss;     // also reduce the YvMoEGate loss (the gate's per-token kernel ran before)
    GateLossArgs loss;
};

// Inclusive prefix sum over the 64 lanes of a wavefront, by DPP moves (no LDS permute round
// trips): shifts right by 1, 2, 4 and 8 lanes inside each row of 16 (lanes without a source
// add 0), then lane 15 of rows 0 and 2 into rows 1 and 3 (row_bcast:15) and lane 31 into rows
// 2 and 3 (row_bcast:31).
__device__ __forceinline__ int wave_incl_scan(int v) {
    v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
    v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
    v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
    v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
    v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
    v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
    return v;
}

// EARLY_LOSS: the launch with the YvMoEGate loss over at most 64 groups (an instance of its own,
// so the other launches keep their registers and schedule).
template <bool EARLY_LOSS>
__global__ __launch_bounds__(1024) void route_small_kernel(SmallRouteArgs a) {
    __shared__ int hist[YVMOE_MAX_EXPERTS];
    __shared__ int s_off[YVMOE_MAX_EXPERTS + 1];
    __shared__ unsigned short cnt[kSmallChunks][YVMOE_MAX_EXPERTS];
    __shared__ unsigned char s_idx[kSmallSlots];
    __shared__ unsigned char s_allowed[kSmallSlots];
    __shared__ unsigned short s_rk[kSmallSlots];
    __shared__ unsigned short s_perm[kSmallSlots];
    __shared__ float s_topp[kSmallSlots];
    __shared__ float s_w0[kSmallSlots];
    __shared__ float s_score[kSmallRouteTok];
    __shared__ float s_tpos[kSmallSlots];          // probability of the slot at each position
    __shared__ unsigned char s_epos[kSmallSlots];  // expert of each position
    __shared__ int s_cap;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    const int N = a.N, E = a.E, k = a.k;
    const int nb = (N + kTokPerBlock - 1) / kTokPerBlock;
    const int nslots = N * k;
    const int nchunks = (nslots + 63) / 64;

    // the YvMoEGate loss: its per-work-group sums sit in the gate's workspace region, which the
    // tile table below may overwrite, so they are read before it is written — at decode sizes
    // (at most 64 groups) their loads go out with this kernel's first ones and the sums run
    // between the routing's own barriers; otherwise the whole loss first
    LossRegs lr;
    if constexpr (EARLY_LOSS) {
        gate_loss_load(a.loss, lr);
    } else if (a.has_loss) {
        gate_loss_block(a.loss);
        __syncthreads();
    }
    for (int q = tid; q < E; q += 1024) hist[q] = 0;
    for (int q = tid; q < nchunks * E; q += 1024) cnt[q / E][q % E] = 0;
    __syncthreads();
    for (int s = tid; s < nslots; s += 1024) {
        const int e = (int)a.indices[s];
        s_idx[s] = (unsigned char)e;
        s_topp[s] = a.topp[s];
        s_w0[s] = a.w0[s];  // read here, with the rest, not at the end
        s_allowed[s] = 1;
        atomicAdd(&hist[e], 1);
    }
    if (a.cap_mode == 2 && tid < kSmallRouteTok) s_score[tid] = tid < N ? a.score[tid] : 0.0f;
    __syncthreads();
    // (the loss partial sums are all read here, before the tile table is written)
    if constexpr (EARLY_LOSS) gate_loss_cols(a.loss, lr);

    // stable scatter, part 1: rank within a 64-slot chunk from 8 ballots over the expert id
    // bits (all waves); counts, offsets and capacity (wave 0, after its chunks)
    for (int c = wave; c < nchunks; c += 16) {
        const int s = c * 64 + lane;
        const bool valid = s < nslots;
        const int e = valid ? (int)s_idx[s] : 0;
        unsigned long long mask = __ballot(valid);
#pragma unroll
        for (int bit = 0; bit < 8; ++bit) {
            const bool on = (e >> bit) & 1;
            const unsigned long long bb = __ballot(valid && on);
            mask &= on ? bb : ~bb;
        }
        const unsigned long long below = mask & ((1ull << lane) - 1ull);
        if (valid) {
            s_rk[s] = (unsigned short)__popcll(below);
            if (below == 0ull) cnt[c][e] = (unsigned short)__popcll(mask);
        }
    }
    if (wave == 0) {
        // lane l owns experts 4l .. 4l + 3 (E <= 256)
        int h[4], loc = 0;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            h[i] = e < E ? hist[e] : 0;
            loc += h[i];
        }
        int run = wave_incl_scan(loc) - loc;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int e = 4 * lane + i;
            if (e < E) {
                a.counts[e] = h[i];
                run += h[i];
                a.offsets[e + 1] = run;
                s_off[e + 1] = run;
            }
        }
        if (lane == 0) {
            a.offsets[0] = 0;
            s_off[0] = 0;
            // complexity sums: per 64-token block in token order (invalid tokens 0), then
            // route_scan_kernel's 1024-wide tree, which for nb <= 4 block sums r0..r3 (the
            // rest 0) reduces to (r0 + r2) + (r1 + r3)
            float r[4] = {0.0f, 0.0f, 0.0f, 0.0f};
            if (a.cap_mode == 2)
                for (int b = 0; b < nb; ++b) {
                    float bs = 0.0f;
                    for (int i = 0; i < kTokPerBlock; ++i) bs = bs + s_score[b * kTokPerBlock + i];
                    r[b] = 0.0f + bs;
                }
            const float total = (r[0] + r[2]) + (r[1] + r[3]);
            int cap = -1;
            if (a.cap_mode == 1) {
                cap = a.cap_explicit;
            } else if (a.cap_mode == 2 || a.cap_mode == 3) {
                double cf = a.cap_factor;
                if (a.cap_mode == 2) {
                    const float avg = total / (float)N;  // complexity_scores.mean() (gate.py:1117)
                    cf = 0.5 + 1.5 * (double)avg;
                    if (cf > 2.0) cf = 2.0;
                    if (cf < 0.5) cf = 0.5;
                }
                cap = (int)((double)N * cf / (double)E);
                if (cap < a.min_cap) cap = a.min_cap;
            }
            *a.cap_out = cap;
            s_cap = cap;
        }
    }
    __syncthreads();

    // stable scatter, part 2: chunk counts prefix-summed per expert, then positions
    if (tid < E) {
        int run = 0;
        for (int c = 0; c < nchunks; ++c) {
            const int v = cnt[c][tid];
            cnt[c][tid] = (unsigned short)run;
            run += v;
        }
    }
    if constexpr (EARLY_LOSS) gate_loss_lb(a.loss);
    __syncthreads();
    for (int s = tid; s < nslots; s += 1024) {
        const int e = s_idx[s];
        const int p = s_off[e] + cnt[s / 64][e] + s_rk[s];
        a.perm[p] = s;
        a.pos[s] = p;
        s_perm[p] = (unsigned short)s;
        s_tpos[p] = s_topp[s];
        s_epos[p] = (unsigned char)e;
    }
    __syncthreads();

    // capacity trim, every position at once: the slot at position p of an over-full expert's
    // segment [off, off + n) (positions in token order: the scatter is stable) is kept iff
    // #{j: p_j > p_p} + #{j before p: p_j == p_p} < cap. The last wavefront builds the tile
    // table meanwhile (it holds positions only when there are more than 960 slots).
    const int cap = s_cap;
    if (cap >= 0) {
        for (int q = tid; q < nslots; q += 1024) {
            const int e = s_epos[q];
            const int off = s_off[e], n = s_off[e + 1] - off;
            if (n <= cap) continue;
            const float tq = s_tpos[q];
            int rank = 0;
            for (int j = 0; j < n; ++j) {
                const float tj = s_tpos[off + j];
                rank += (tj > tq || (tj == tq && off + j < q)) ? 1 : 0;
            }
            if (rank >= cap) s_allowed[s_perm[q]] = 0;
        }
    }
    if (wave == 15 && a.tiles.seg != nullptr) {
        // tile table of the expert GEMMs (build_tiles_kernel): lane l owns segments 5l .. 5l + 4
        const int S = a.tiles.S, tr = a.tiles.tile_rows, fold = a.tiles.fold;
        const int lg = 31 - __builtin_clz(tr);  // tile heights are powers of two (host-checked)
        const int nseg = E + S;
        int s0[5], nt[5], loc = 0;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int sg = 5 * lane + i;
            int b = 0, e_ = 0;
            if (sg < nseg) {
                if (sg < E) {
                    b = s_off[sg];
                    e_ = s_off[sg + 1];
                } else {
                    b = N * k + (sg - E) * N;
                    e_ = b + N;
                }
                a.tiles.seg[sg] = b;
                if (sg == nseg - 1) a.tiles.seg[nseg] = e_;
            }
            s0[i] = b;
            const int rows = e_ - b, full = rows >> lg, rem = rows & (tr - 1);
            nt[i] = full + ((rem > 0 && !(full > 0 && rem <= fold)) ? 1 : 0);  // seg_tiles
            loc += nt[i];
        }
        const int incl = wave_incl_scan(loc);
        int start = incl - loc;
#pragma unroll
        for (int i = 0; i < 5; ++i) {
            const int sg = 5 * lane + i;
            for (int q = 0; q < nt[i]; ++q) {
                a.tiles.tile_seg[start + q] = sg;
                a.tiles.tile_row0[start + q] = s0[i] + q * tr;
            }
            start += nt[i];
        }
        if (lane == 63) *a.tiles.ntiles = incl;
    }
    __syncthreads();

    // weights: renormalised over the kept slots (renorm_kernel), or the first softmax
    // unchanged in fixed-shape mode; the loss by the last thread (at most 256 tokens here)
    if constexpr (EARLY_LOSS) {
        if (tid == 1023) gate_loss_total(a.loss);
    }
    if (tid < N) {
        const int t = tid;
        if (a.cap_mode != 0) {
            float tmp[YVMOE_MAX_TOPK];
            float tot = 0.0f;
            for (int j = 0; j < k; ++j) {
                const int s = t * k + j;
                tmp[j] = s_w0[s] * (s_allowed[s] ? 1.0f : 0.0f);
                tot = tot + tmp[j];
            }
            const float den = tot > 1e-8f ? tot : 1e-8f;
            const float keep = tot > 0.0f ? 1.0f : 0.0f;
            for (int j = 0; j < k; ++j) a.weights[t * k + j] = (tmp[j] * keep) / den;
        } else {
            for (int j = 0; j < k; ++j) a.weights[t * k + j] = s_w0[t * k + j];
        }
    }
}

// The YvMoEGate loss after a routing that does not end in route_small_kernel.
__global__ __launch_bounds__(1024) void route_gate_loss_kernel(GateLossArgs a) { gate_loss_block(a); }

// ------------------------------------------------------------------ external routing
// The dispatch entry (PiscesLxFusedMoEDispatch.forward, opss/infer/fused_moe.py:69-100) takes
// the routing from its caller. One block per 64 tokens: the block's histogram of expert ids
// in [0, E) and its count of ids outside that range (those slots are left out of the
// permutation and the combine; the entry reports how many there were), and with w32 set the
// bf16 routing weights widened to fp32 (exact).
__global__ __launch_bounds__(256) void dispatch_hist_kernel(
    const int64_t* __restrict__ idx, const unsigned short* __restrict__ w_bf16, int N, int E, int k,
    float* __restrict__ w32, int* __restrict__ blockhist, int* __restrict__ blockinv) {
    __shared__ int hist[YVMOE_MAX_EXPERTS];
    __shared__ int s_inv;
    const int tid = threadIdx.x;
    for (int e = tid; e < E; e += 256) hist[e] = 0;
    if (tid == 0) s_inv = 0;
    __syncthreads();
    const long long base = (long long)blockIdx.x * kTokPerBlock * k;
    const long long total = (long long)N * k;
    const long long span = total - base < (long long)kTokPerBlock * k ? total - base
                                                                      : (long long)kTokPerBlock * k;
    const int nslots = (int)span;
    int inv = 0;
    for (int s = tid; s < nslots; s += 256) {
        const long long q = base + s;
        const long long v = idx[q];
        if (v >= 0 && v < E) atomicAdd(&hist[(int)v], 1);
        else ++inv;
        if (w32 != nullptr) w32[q] = __uint_as_float((unsigned)w_bf16[q] << 16);
    }
    if (inv) atomicAdd(&s_inv, inv);
    __syncthreads();
    for (int e = tid; e < E; e += 256) blockhist[(size_t)blockIdx.x * E + e] = hist[e];
    if (tid == 0) blockinv[blockIdx.x] = s_inv;
}

}  // namespace

int dispatch_route_launch(const int64_t* idx, const unsigned short* w_bf16, float* w32, int N,
                          int E, int k, int* counts, int* offsets, int* perm, int* pos,
                          int* invalid, int* cap_scratch, char* ws, hipStream_t st) {
    const RouteWs L = route_ws(N, E, k);
    int* blockhist = (int*)(ws + L.blockhist);
    int* blockoff = (int*)(ws + L.blockoff);
    int* blockinv = (int*)(ws + L.blocksum);  // the complexity sums' region: [nb] 4-byte slots
    const int nb = ceil_div(N, kTokPerBlock);
    if (N > 0) {
        dispatch_hist_kernel<<<nb, 256, 0, st>>>(idx, w_bf16, N, E, k, w32, blockhist, blockinv);
        YV_LAUNCH_CHECK("dispatch_hist");
    }
    route_scan_kernel<<<1, 1024, 0, st>>>(blockhist, nb, E, N, nullptr, 0, -1, 0, 1.0, counts,
                                            offsets, blockoff, cap_scratch, blockinv, invalid);
    YV_LAUNCH_CHECK("dispatch_scan");
    if (N > 0) {
        route_scatter_kernel<int64_t><<<nb, 256, 0, st>>>(idx, N, E, k, blockoff, perm, pos);
        YV_LAUNCH_CHECK("dispatch_scatter");
    }
    return YVMOE_OK;
}

GateTopk route_topk_outputs(int N, int E, int k, yvmoe_routing* out, char* ws) {
    const RouteWs L = route_ws(N, E, k);
    return GateTopk{out->indices, (float*)(ws + L.topp), (float*)(ws + L.w0), k};
}

int route_launch(const float* logits, int ld, const float* pred, int pred_ld, int N,
                 const yvmoe_router* r, int cap_override, yvmoe_routing* out, char* ws,
                 hipStream_t st, int ksplit, long long split_stride, const TileTable* tiles,
                 bool topk_ready, const GateLossArgs* loss) {
    const int E = r->num_experts, k = r->top_k;
    const RouteWs L = route_ws(N, E, k);
    float* topp = (float*)(ws + L.topp);
    float* w0 = (float*)(ws + L.w0);
    uint8_t* allowed = (uint8_t*)(ws + L.allowed);
    int* blockhist = (int*)(ws + L.blockhist);
    int* blockoff = (int*)(ws + L.blockoff);
    float* blocksum = (float*)(ws + L.blocksum);
    const int nb = ceil_div(N, kTokPerBlock);
    const bool fixed = r->fixed_shape_mode != 0;
    int cap_mode = 0;
    if (!fixed) cap_mode = cap_override >= 0 ? 1 : (r->dynamic_capacity ? 2 : 3);
    const float* use_pred = (cap_mode == 2) ? pred : nullptr;
    YV_REQUIRE(cap_mode != 2 || pred != nullptr, YVMOE_ERR_ARG,
               "dynamic capacity needs the complexity predictor columns (or a capacity override)");
    const int pred_terms = (pred_ld - pad16(E)) / kPredDim;
    const bool small_path = N > 0 && N <= kSmallRouteTok && (use_pred == nullptr || pred_terms <= kMaxPredTerms);
    YV_REQUIRE(!topk_ready || (small_path && cap_mode != 2), YVMOE_ERR_ARG,
               "internal: ready top-k outputs need the small-batch path without dynamic capacity");
    if (small_path) {
        float* score = (float*)(ws + L.score);
        const float* lpred = use_pred;
        if (!topk_ready) {
#define YV_TOPKS(NVV)                                                                              \
    route_topk_small_kernel<NVV><<<N, 256, 0, st>>>(                                                \
        logits, lpred, ld, ksplit, split_stride, pred_terms, r->bias, r->b1, r->w2, r->b2, N, E, k, \
        out->indices, topp, w0, score)
        if (E <= 16) YV_TOPKS(1);
        else if (E <= 64) YV_TOPKS(4);
        else if (E <= 128) YV_TOPKS(8);
        else YV_TOPKS(16);
#undef YV_TOPKS
        YV_LAUNCH_CHECK("route_topk_small");
        }
        SmallRouteArgs a{};
        a.N = N;
        a.E = E;
        a.k = k;
        a.cap_mode = cap_mode;
        a.cap_explicit = cap_override;
        a.min_cap = r->min_capacity;
        a.cap_factor = r->capacity_factor;
        a.indices = out->indices;
        a.topp = topp;
        a.w0 = w0;
        a.score = score;
        a.weights = out->weights;
        a.counts = out->counts;
        a.offsets = out->offsets;
        a.perm = out->perm;
        a.pos = out->pos;
        a.cap_out = out->capacity;
        if (tiles) {
            YV_REQUIRE(tiles->tile_rows > 0 && (tiles->tile_rows & (tiles->tile_rows - 1)) == 0,
                       YVMOE_ERR_ARG, "tile rows %d not a power of two", tiles->tile_rows);
            YV_REQUIRE(tiles->light == 0, YVMOE_ERR_ARG, "internal: light tile tables are built by the FFN");
            a.tiles = *tiles;
        }
        if (loss != nullptr) {
            a.has_loss = 1;
            a.loss = *loss;
        }
        if (a.has_loss && a.loss.G <= 64)
            route_small_kernel<true><<<1, 1024, 0, st>>>(a);
        else
            route_small_kernel<false><<<1, 1024, 0, st>>>(a);
        YV_LAUNCH_CHECK("route_small");
        return YVMOE_OK;
    }
    if (loss != nullptr) {
        route_gate_loss_kernel<<<1, 1024, 0, st>>>(*loss);
        YV_LAUNCH_CHECK("route_gate_loss");
    }
    YV_REQUIRE(tiles == nullptr, YVMOE_ERR_ARG, "internal: tile building is for small batches only");
    YV_REQUIRE(ksplit >= 1 && ksplit <= kFoldSplits, YVMOE_ERR_ARG,
               "internal: the top-k kernel sums at most %d split partial sums (got %d)", kFoldSplits, ksplit);
    if (N == 0) {
        route_scan_kernel<<<1, 1024, 0, st>>>(blockhist, 0, E, 0, blocksum, cap_mode,
                                                cap_override, r->min_capacity,
                                                r->capacity_factor, out->counts, out->offsets,
                                                blockoff, out->capacity);
        YV_LAUNCH_CHECK("route_scan");
        return YVMOE_OK;
    }
    // fixed mode has no trim: the top-k kernel's weights are the final ones
    float* wdst = fixed ? out->weights : w0;
#define YV_TOPK(NVV)                                                                        \
    route_topk_kernel<NVV><<<nb, 1024, 0, st>>>(logits, ld, r->bias, use_pred, pred_ld,      \
                                                pred_terms, r->b1, r->w2, r->b2, N, E, k,    \
                                                out->indices, topp, wdst, allowed, blockhist, \
                                                blocksum, ksplit, split_stride)
    if (E <= 16) YV_TOPK(1);
    else if (E <= 64) YV_TOPK(4);
    else if (E <= 128) YV_TOPK(8);
    else YV_TOPK(16);
#undef YV_TOPK
    YV_LAUNCH_CHECK("route_topk");
    route_scan_kernel<<<1, 1024, 0, st>>>(blockhist, nb, E, N, blocksum, cap_mode, cap_override,
                                            r->min_capacity, r->capacity_factor, out->counts,
                                            out->offsets, blockoff, out->capacity);
    YV_LAUNCH_CHECK("route_scan");
    route_scatter_kernel<int64_t><<<nb, 256, 0, st>>>(out->indices, N, E, k, blockoff, out->perm,
                                                      out->pos);
    YV_LAUNCH_CHECK("route_scatter");
    if (!fixed) {
        capacity_trim_kernel<<<E, 256, 0, st>>>(out->counts, out->offsets, out->capacity,
                                                out->perm, topp, allowed);
        YV_LAUNCH_CHECK("capacity_trim");
        renorm_kernel<<<ceil_div(N, 256), 256, 0, st>>>(w0, allowed, N, k, out->weights);
        YV_LAUNCH_CHECK("renorm");
    }
    return YVMOE_OK;
}

}  // namespace yvmoe
