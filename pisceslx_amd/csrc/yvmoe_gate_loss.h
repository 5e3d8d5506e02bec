// YvMoEGate loss from per-work-group sums (model/moe/gate.py:433-444, :556-610):
//   loss = alpha · Σ_e (mean_n score_e - 1/E)² + capacity term + z_alpha · mean(logits²)
//          + 0.01 · (mean_n Σ_e soft - budget)²
// part holds E + 2 columns of G per-work-group sums (scores per expert, Σ logits², Σ soft).
// Run by one work-group of 1024 threads: its own kernel after the per-token kernels
// (yvmoe_moegate.hip), or the tail of the small-batch routing kernel (yvmoe_route.hip), which
// runs next on the stream at decode sizes — the same arithmetic either way. Column c is summed
// by P threads (contiguous group ranges, 32 loads in flight each) and the P partial sums in
// order; the load-balance sum over experts is one wave reduction per wave and the waves in
// order.
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
    __shared__ float psum[1024];
    __shared__ float col[YVMOE_MAX_EXPERTS + 2];
    __shared__ float red[16];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int E = a.E, G = a.G;
    int cp = 1;
    while (cp < E + 2) cp <<= 1;
    const int P = 1024 / cp;  // threads per column (>= 2: E + 2 <= 258)
    const int c = tid / P, p = tid % P;
    const int chunk = (G + P - 1) / P;
    float sum = 0.f;
    if (c < E + 2) {
        const float* pc = a.part + (long long)c * G;
        const int g1 = min(G, (p + 1) * chunk);
        for (int g0 = p * chunk; g0 < g1; g0 += 32) {
            float v[32];
#pragma unroll
            for (int i = 0; i < 32; ++i) v[i] = g0 + i < g1 ? pc[g0 + i] : 0.f;
#pragma unroll
            for (int i = 0; i < 32; ++i) sum += v[i];
        }
    }
    psum[tid] = sum;
    __syncthreads();
    if (tid < E + 2) {
        float s = psum[tid * P];
        for (int i = 1; i < P; ++i) s += psum[tid * P + i];
        col[tid] = s;
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

}  // namespace
}  // namespace yvmoe
