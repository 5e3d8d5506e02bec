// Softmax and top-k of one token (YvStableMoEGate / YvMoEGate routing, model/moe/gate.py:
// 1212-1223 and :405-416): the bit-exact arithmetic shared by the routing kernels
// (yvmoe_route.hip) and the YvMoEGate per-token kernel (yvmoe_moegate.hip), which routes its
// own tokens at decode sizes. The CPU oracle (oracle/route_oracle.c) follows the same
// specification: Cody-Waite exp with the Cephes ln2 split and a degree-7 Taylor polynomial,
// 16-lane butterfly sums, an IEEE divide, top-k by (p desc, index asc). No multiply-add is
// fused in these functions whatever the including file's flags (the pragmas below), and the
// including file is built with the correctly rounded fp32 divide.
#pragma once

#include <hip/hip_runtime.h>

namespace yvmoe {
namespace {

constexpr int kLanes = 16;  // lanes cooperating on one token

__device__ __forceinline__ float yv_expf_core(float x) {
#pragma clang fp contract(off)
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

__device__ __forceinline__ float yv_expf(float x) {
#pragma clang fp contract(off)
    // the out-of-range results by selects rather than early returns (no branches); the clamped
    // argument keeps the core's arithmetic finite, and its result is discarded for those inputs
    const float xc = fminf(fmaxf(x, -86.0f), 88.0f);
    const float r0 = yv_expf_core(xc);
    return !(x >= -86.0f) ? 0.0f : (x > 88.0f ? __builtin_huge_valf() : r0);
}

// Value of lane (l + o) % 16 of this lane's 16-lane row (DPP row_ror, a VALU move instead of
// an LDS permute). A butterfly over o = 8, 4, 2, 1 with rotations combines the same operand
// values as the xor butterfly: after the step with o, every partial is periodic with period
// o, so lane l's rotation partner holds the same bits as its xor partner l ^ o. Sums and
// maxima are therefore bit-identical to the xor form.
template <int O>
__device__ __forceinline__ int rot16(int v) {
    return __builtin_amdgcn_update_dpp(0, v, 0x120 + O, 0xf, 0xf, false);
}
template <int O>
__device__ __forceinline__ float rot16(float v) {
    return __int_as_float(rot16<O>(__float_as_int(v)));
}
#define YV_BFLY16(STEP) do { STEP(8); STEP(4); STEP(2); STEP(1); } while (0)

// Softmax and top-k of one token by its 16 lanes (lane l holds experts l, l + 16, ...).
// logit(e) returns the fp32 logit of expert e. Lane j < k ends with the j-th choice: expert
// id, its probability and its first-softmax weight exp(p_j - p_0) / sum.
template <int NV, typename LogitFn>
__device__ __forceinline__ void topk_token(LogitFn logit, const float* __restrict__ bias, int l, int E,
                                           int k, int& my_id, float& my_ts, float& my_w0) {
#pragma clang fp contract(off)
    float z[NV];
    float m = -__builtin_huge_valf();
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int e = l + kLanes * i;
        z[i] = 0.0f;
        if (e < E) {
            float v = logit(e);
            if (bias) v = v + bias[e];
            z[i] = v;
            if (v > m) m = v;
        }
    }
#define YV_MAXSTEP(O)                    \
    do {                                 \
        const float mo = rot16<O>(m);    \
        if (mo > m) m = mo;              \
    } while (0)
    YV_BFLY16(YV_MAXSTEP);
#undef YV_MAXSTEP
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int e = l + kLanes * i;
        if (e < E) {
            z[i] = yv_expf(z[i] - m);
            part = part + z[i];
        }
    }
#define YV_SUMSTEP(O) part = part + rot16<O>(part)
    YV_BFLY16(YV_SUMSTEP);
#undef YV_SUMSTEP
#pragma unroll
    for (int i = 0; i < NV; ++i) z[i] = z[i] / part;

    // top-k by (p desc, index asc). Each candidate is one 64-bit key, the probability's bits
    // high (non-negative floats order like their bits) and the inverted expert index low (the
    // lower index wins a tie), so an argmax step is one unsigned compare and two selects
    // instead of the short-circuit float-and-index test, whose branches cost more than the
    // arithmetic. Taken, out-of-range and NaN entries hold key 0, below every candidate (a
    // NaN probability was never better than anything, so it was never chosen either).
    unsigned long long key[NV];
#pragma unroll
    for (int i = 0; i < NV; ++i) {
        const int e = l + kLanes * i;
        key[i] = (e < E && z[i] == z[i])
                     ? ((unsigned long long)__float_as_uint(z[i]) << 32) | (unsigned)(~e)
                     : 0ull;
    }
    float e0 = 0.0f, ts0 = 0.0f, tot = 0.0f;
    my_ts = 0.0f;
    my_id = 0;
    for (int j = 0; j < k; ++j) {
        unsigned long long b = key[0];
#pragma unroll
        for (int i = 1; i < NV; ++i) b = key[i] > b ? key[i] : b;
#define YV_KEYSTEP(O)                                                                           \
    do {                                                                                        \
        const unsigned lo = (unsigned)rot16<O>((int)(unsigned)b);                               \
        const unsigned hi = (unsigned)rot16<O>((int)(unsigned)(b >> 32));                       \
        const unsigned long long o = ((unsigned long long)hi << 32) | lo;                       \
        b = o > b ? o : b;                                                                      \
    } while (0)
        YV_BFLY16(YV_KEYSTEP);
#undef YV_KEYSTEP
        // no candidate left (only with NaN probabilities): probability -1, index INT_MAX
        const float bv = b != 0ull ? __uint_as_float((unsigned)(b >> 32)) : -1.0f;
        const int be = b != 0ull ? (int)~(unsigned)b : 0x7fffffff;
#pragma unroll
        for (int i = 0; i < NV; ++i) key[i] = key[i] == b ? 0ull : key[i];  // the owner takes it
        if (j == 0) ts0 = bv;
        const float ej = yv_expf(bv - ts0);
        tot = tot + ej;
        if (l == j) {
            my_ts = bv;
            my_id = be;
            e0 = ej;
        }
    }
    my_w0 = e0 / tot;
}

}  // namespace
}  // namespace yvmoe
