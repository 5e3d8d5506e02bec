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

namespace yvmoe {
namespace {

constexpr int kLanes = 16;  // lanes cooperating on one token

__device__ __forceinline__ float yv_expf(float x) {
    if (!(x >= -86.0f)) return 0.0f;
    if (x > 88.0f) return __builtin_huge_valf();
    float fn = rintf(x * 1.44269504088896341f);
    int n = (int)fn;
    float r = x - fn * 0.693359375f;
    r = r + fn * 2.12194440e-4f;
    float p = 1.98412698e-4f;
    p = p * r + 1.38888889e-3f;
    p = p * r + 8.33333333e-3f;
    p = p * r + 4.16666667e-2f;
    p = p * r + 1.66666667e-1f;
    p = p * r + 0.5f;
    p = p * r + 1.0f;
    p = p * r + 1.0f;
    return p * __uint_as_float((unsigned)(n + 127) << 23);
}

__device__ __forceinline__ bool better(float v1, int e1, float v2, int e2) {
    return v1 > v2 || (v1 == v2 && e1 < e2);
}

// One block = 64 tokens, 16 lanes per token, all 64 tokens in one pass (1024 threads).
template <int NV>
__global__ __launch_bounds__(1024) void route_topk_kernel(
    const float* __restrict__ logits, int ld, const float* __restrict__ bias,
    const float* __restrict__ pred, int pred_ld, int pred_terms, const float* __restrict__ b1,
    const float* __restrict__ w2, const float* __restrict__ b2, int N, int E, int k,
    int64_t* __restrict__ idx_out, float* __restrict__ topp, float* __restrict__ w0,
    uint8_t* __restrict__ allowed, int* __restrict__ blockhist, float* __restrict__ blocksum) {
    __shared__ int hist[YVMOE_MAX_EXPERTS];
    __shared__ float score[kTokPerBlock];
    const int tid = threadIdx.x;
    const int g = tid / kLanes;
    const int l = tid % kLanes;
    for (int e = tid; e < E; e += blockDim.x) hist[e] = 0;
    if (tid < kTokPerBlock) score[tid] = 0.0f;
    __syncthreads();

    {
        const int tl = g;
        const int t = blockIdx.x * kTokPerBlock + tl;
        if (t < N) {  // uniform across the 16 lanes of a token
            float z[NV];
            float m = -__builtin_huge_valf();
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int e = l + kLanes * i;
                z[i] = 0.0f;
                if (e < E) {
                    float v = logits[(size_t)t * ld + e];
                    if (bias) v = v + bias[e];
                    z[i] = v;
                    if (v > m) m = v;
                }
            }
#pragma unroll
            for (int o = kLanes / 2; o >= 1; o >>= 1) {
                float mo = __shfl_xor(m, o, kLanes);
                if (mo > m) m = mo;
            }
            float part = 0.0f;
#pragma unroll
            for (int i = 0; i < NV; ++i) {
                const int e = l + kLanes * i;
                if (e < E) {
                    z[i] = yv_expf(z[i] - m);
                    part = part + z[i];
                }
            }
#pragma unroll
            for (int o = kLanes / 2; o >= 1; o >>= 1) part = part + __shfl_xor(part, o, kLanes);
#pragma unroll
            for (int i = 0; i < NV; ++i) z[i] = z[i] / part;

            // top-k by (p desc, index asc)
            unsigned taken = 0u;
            float my_ts = 0.0f, my_e0 = 0.0f, ts0 = 0.0f, tot = 0.0f;
            int my_id = 0;
            for (int j = 0; j < k; ++j) {
                float bv = -1.0f;
                int be = 0x7fffffff;
                int bi = -1;
#pragma unroll
                for (int i = 0; i < NV; ++i) {
                    const int e = l + kLanes * i;
                    if (e < E && !((taken >> i) & 1u) && better(z[i], e, bv, be)) {
                        bv = z[i];
                        be = e;
                        bi = i;
                    }
                }
#pragma unroll
                for (int o = kLanes / 2; o >= 1; o >>= 1) {
                    float ov = __shfl_xor(bv, o, kLanes);
                    int oe = __shfl_xor(be, o, kLanes);
                    if (better(ov, oe, bv, be)) {
                        bv = ov;
                        be = oe;
                    }
                }
                if ((be % kLanes) == l && bi >= 0 && (l + kLanes * bi) == be) taken |= 1u << bi;
                if (j == 0) ts0 = bv;
                const float ej = yv_expf(bv - ts0);
                tot = tot + ej;
                if (l == j) {
                    my_ts = bv;
                    my_id = be;
                    my_e0 = ej;
                }
            }
            if (l < k) {
                const size_t s = (size_t)t * k + l;
                idx_out[s] = (int64_t)my_id;
                topp[s] = my_ts;
                w0[s] = my_e0 / tot;
                allowed[s] = 1;
                atomicAdd(&hist[my_id], 1);
            }
            if (pred != nullptr) {
                // complexity_predictor: sigmoid(w2 . relu(W1 x + b1) + b2)  (gate.py:930-936)
                float acc = 0.0f;
#pragma unroll
                for (int i = 0; i < kPredDim / kLanes; ++i) {
                    const int c = l + kLanes * i;
                    float hsum = 0.0f;
                    for (int q = 0; q < pred_terms; ++q)
                        hsum = hsum + pred[(size_t)t * pred_ld + q * kPredDim + c];
                    hsum = hsum + b1[c];
                    hsum = hsum > 0.0f ? hsum : 0.0f;
                    acc = acc + w2[c] * hsum;
                }
#pragma unroll
                for (int o = kLanes / 2; o >= 1; o >>= 1) acc = acc + __shfl_xor(acc, o, kLanes);
                if (l == 0) score[tl] = 1.0f / (1.0f + expf(-(acc + b2[0])));
            }
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
__global__ __launch_bounds__(1024) void route_scan_kernel(
    const int* __restrict__ blockhist, int nb, int E, int N, const float* __restrict__ blocksum,
    int cap_mode, int cap_explicit, int min_cap, double cap_factor, int* __restrict__ counts,
    int* __restrict__ offsets, int* __restrict__ blockoff, int* __restrict__ cap_out) {
    __shared__ int part[1024];
    __shared__ int scan[YVMOE_MAX_EXPERTS];
    __shared__ float red[1024];
    const int tid = threadIdx.x;
    const int C = 1024 / E;  // chunks of blocks per expert (E <= 256 -> C >= 4)
    const int e = tid % E;
    const int c = tid / E;
    const bool active = c < C;
    int b0 = 0, b1 = 0;
    if (active) {
        b0 = (int)((long long)c * nb / C);
        b1 = (int)((long long)(c + 1) * nb / C);
        int s = 0;
        for (int b = b0; b < b1; ++b) s += blockhist[(size_t)b * E + e];
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
    if (tid < E) offsets[tid + 1] = scan[tid];
    if (tid == 0) {
        offsets[0] = 0;
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
// its 64-slot chunk comes from 8 wavefront ballots over the expert id bits.
__global__ __launch_bounds__(256) void route_scatter_kernel(
    const int64_t* __restrict__ idx, int N, int E, int k, const int* __restrict__ blockoff,
    int* __restrict__ perm, int* __restrict__ pos, int* __restrict__ tok) {
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
    for (int q = tid; q < nchunks * E; q += 256) cnt[q / E][q % E] = 0;
    __syncthreads();
    for (int c = wave; c < nchunks; c += 4) {
        const int s = c * 64 + lane;
        const bool valid = s < nslots;
        const int e = valid ? (int)idx[base + s] : 0;
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
        const int e = (int)idx[base + s];
        const int p = blockoff[(size_t)blockIdx.x * E + e] + cnt[s / 64][e] + rk[s];
        const long long slot = base + s;
        perm[p] = (int)slot;
        pos[slot] = p;
        tok[p] = (int)(slot / k);
    }
}

// Capacity trim of one expert: LDS radix select of the cap-th largest p (4 passes of 8
// bits on the fp32 bit pattern, which orders like the value for p >= 0), then keep
// p > T and the first (cap - #{p > T}) slots with p == T in token order (gate.py:1228-1236).
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
    unsigned prefix = 0u, pmask = 0u;
    int rem = cap;
    for (int shift = 24; shift >= 0; shift -= 8) {
        hist[tid] = 0u;
        __syncthreads();
        for (int i = tid; i < n; i += 256) {
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
    for (int b = 0; b < n; b += 256) {
        const int i = b + tid;
        const bool valid = i < n;
        int slot = -1;
        unsigned key = 0u;
        if (valid) {
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

__global__ void copy_f32_kernel(const float* __restrict__ a, float* __restrict__ b, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) b[i] = a[i];
}

}  // namespace

int route_launch(const float* logits, int ld, const float* pred, int pred_ld, int N,
                 const yvmoe_router* r, int cap_override, yvmoe_routing* out, char* ws,
                 hipStream_t st) {
    const int E = r->num_experts, k = r->top_k;
    const RouteWs L = route_ws(N, E, k);
    float* topp = (float*)(ws + L.topp);
    float* w0 = (float*)(ws + L.w0);
    uint8_t* allowed = (uint8_t*)(ws + L.allowed);
    int* blockhist = (int*)(ws + L.blockhist);
    int* blockoff = (int*)(ws + L.blockoff);
    float* blocksum = (float*)(ws + L.blocksum);
    int* tok = (int*)(ws + L.tok);
    const int nb = ceil_div(N, kTokPerBlock);
    const bool fixed = r->fixed_shape_mode != 0;
    int cap_mode = 0;
    if (!fixed) cap_mode = cap_override >= 0 ? 1 : (r->dynamic_capacity ? 2 : 3);
    const float* use_pred = (cap_mode == 2) ? pred : nullptr;
    YV_REQUIRE(cap_mode != 2 || pred != nullptr, YVMOE_ERR_ARG,
               "dynamic capacity needs the complexity predictor columns (or a capacity override)");
    const int pred_terms = (pred_ld - pad16(E)) / kPredDim;
    if (N == 0) {
        route_scan_kernel<<<1, 1024, 0, st>>>(blockhist, 0, E, 0, blocksum, cap_mode,
                                                cap_override, r->min_capacity,
                                                r->capacity_factor, out->counts, out->offsets,
                                                blockoff, out->capacity);
        YV_LAUNCH_CHECK("route_scan");
        return YVMOE_OK;
    }
#define YV_TOPK(NVV)                                                                        \
    route_topk_kernel<NVV><<<nb, 1024, 0, st>>>(logits, ld, r->bias, use_pred, pred_ld,      \
                                                pred_terms, r->b1, r->w2, r->b2, N, E, k,    \
                                                out->indices, topp, w0, allowed, blockhist, \
                                                blocksum)
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
    route_scatter_kernel<<<nb, 256, 0, st>>>(out->indices, N, E, k, blockoff, out->perm,
                                             out->pos, tok);
    YV_LAUNCH_CHECK("route_scatter");
    if (!fixed) {
        capacity_trim_kernel<<<E, 256, 0, st>>>(out->counts, out->offsets, out->capacity,
                                                out->perm, topp, allowed);
        YV_LAUNCH_CHECK("capacity_trim");
        renorm_kernel<<<ceil_div(N, 256), 256, 0, st>>>(w0, allowed, N, k, out->weights);
        YV_LAUNCH_CHECK("renorm");
    } else {
        const int n = N * k;
        copy_f32_kernel<<<ceil_div(n, 256), 256, 0, st>>>(w0, out->weights, n);
        YV_LAUNCH_CHECK("copy_weights");
    }
    return YVMOE_OK;
}

}  // namespace yvmoe
