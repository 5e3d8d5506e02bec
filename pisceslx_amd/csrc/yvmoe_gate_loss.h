// YvMoEGate loss from per-work-group sums (model/moe/gate.py:433-444, :556-610):
//   loss = alpha · Σ_e (mean_n score_e - 1/E)² + capacity term + z_alpha · mean(logits²)
//          + 0.01 · (mean_n Σ_e soft - budget)²
// part holds E + 2 columns of G per-work-group sums (scores per expert, Σ logits², Σ soft).
// Run by one work-group of 1024 threads: its own kernel after the per-token kernels
// (yvmoe_moegate.hip), or inside the small-batch routing kernel (yvmoe_route.hip), which
// runs next on the stream at decode sizes — the same arithmetic either way. Column c is summed
// by one wavefront (lane l takes groups l, l + 64, ... in order, then a wave reduction: the
// loads of a step are one coalesced 256-byte row; the earlier layout, P threads per column over
// contiguous group ranges, made every load touch 64 cache lines and took 35 us at 1024 groups);
// the load-balance sum over experts is one wave reduction per wave and the waves in order.
#pragma once

#include <hip/hip_runtime.h>

#include "yvmoe_internal.h"

namespace yvmoe {
namespace {

template <int O>
__device__ __forceinline__ float gl_ror16(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + O, 0xf, 0xf, false));
}
__device__ __forceinline__ float gl_wave_sum(float v) {
    v = v + gl_ror16<8>(v);
    v = v + gl_ror16<4>(v);
    v = v + gl_ror16<2>(v);
    v = v + gl_ror16<1>(v);
    auto at = [&](int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); };
    return ((at(0) + at(16)) + at(32)) + at(48);
}

// Every thread of the 1024-thread work-group calls this (it holds barriers).
__device__ __forceinline__ void gate_loss_block(const GateLossArgs& a) {
    __shared__ float col[YVMOE_MAX_EXPERTS + 2];
    __shared__ float red[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E, G = a.G;
    // column c by wavefront c % 16: lane l sums groups l, l + 64, ... in order (coalesced
    // loads, 16 in flight), then the wave reduction
    for (int c = wave; c < E + 2; c += 16) {
        const float* pc = a.part + (long long)c * G;
        float sum = 0.f;
        for (int g0 = 0; g0 < G; g0 += 64 * 16) {
            float v[16];
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int g = g0 + 64 * i + lane;
                v[i] = g < G ? pc[g] : 0.f;
            }
#pragma unroll
            for (int i = 0; i < 16; ++i) sum += v[i];
        }
        sum = gl_wave_sum(sum);
        if (lane == 0) col[c] = sum;
    }
    __syncthreads();
    const float fn = (float)a.N;
    float d = 0.f;
    if (tid < E) {
        d = col[tid] / fn - 1.f / (float)E;
        d = d * d;
    }
    d = gl_wave_sum(d);
    if (lane == 0) red[wave] = d;
    __syncthreads();
    if (tid == 0) {
        float lb = red[0];
        for (int w = 1; w < 16; ++w) lb += red[w];
        float total = a.lb_alpha * lb + a.cap_loss + a.z_alpha * (col[E] / ((float)a.N * (float)E));
        if (a.has_soft) {
            const float ac = col[E + 1] / fn - a.budget;
            total += 0.01f * (ac * ac);
        }
        a.loss[0] = total;
    }
}

// Split form of gate_loss_block for at most 64 groups (the small-batch routing kernel), its
// phases placed between the caller's own barriers: gate_loss_load issues the loads with the
// caller's first loads (lane l of wavefront w holds group l of columns w, w + 16, ...);
// gate_loss_cols (after a barrier that follows the loads; every thread) sums the columns into
// LDS; gate_loss_lb (after a later barrier; every thread) adds the load-balance terms per
// wavefront; gate_loss_total (after a later barrier; one thread) writes the loss. The arithmetic
// is gate_loss_block's: each column's sum is 0 + its lane's value (gate_loss_block's further
// terms are zeros at this size), then the same wave reductions and the waves in order.
constexpr int kLossCols = (YVMOE_MAX_EXPERTS + 2 + 15) / 16;
struct LossRegs {
    float v[kLossCols];
};
struct LossLds {
    float col[YVMOE_MAX_EXPERTS + 2];
    float red[16];
};
__device__ __forceinline__ LossLds& loss_lds() {
    __shared__ LossLds s;
    return s;
}
__device__ __forceinline__ void gate_loss_load(const GateLossArgs& a, LossRegs& r) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < kLossCols; ++i) {
        const int c = wave + 16 * i;
        r.v[i] = (c < a.E + 2 && lane < a.G) ? a.part[(long long)c * a.G + lane] : 0.f;
    }
}
__device__ __forceinline__ void gate_loss_cols(const GateLossArgs& a, const LossRegs& r) {
    LossLds& l = loss_lds();
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int i = 0; i < kLossCols; ++i) {
        const int c = wave + 16 * i;
        if (c < a.E + 2) {
            float sum = 0.f;
            sum += r.v[i];
            sum = gl_wave_sum(sum);
            if (lane == 0) l.col[c] = sum;
        }
    }
}
__device__ __forceinline__ void gate_loss_lb(const GateLossArgs& a) {
    LossLds& l = loss_lds();
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E;
    float d = 0.f;
    if (tid < E) {
        d = l.col[tid] / (float)a.N - 1.f / (float)E;
        d = d * d;
    }
    d = gl_wave_sum(d);
    if (lane == 0) l.red[wave] = d;
}
__device__ __forceinline__ void gate_loss_total(const GateLossArgs& a) {
    const LossLds& l = loss_lds();
    const int E = a.E;
    const float fn = (float)a.N;
    float lb = l.red[0];
    for (int w = 1; w < 16; ++w) lb += l.red[w];
    float total = a.lb_alpha * lb + a.cap_loss + a.z_alpha * (l.col[E] / ((float)a.N * (float)E));
    if (a.has_soft) {
        const float ac = l.col[E + 1] / fn - a.budget;
        total += 0.01f * (ac * ac);
    }
    a.loss[0] = total;
}

}  // namespace
}  // namespace yvmoe
