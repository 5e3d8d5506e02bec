// RMSNorm of the MoE input (model/core/norms.py:178-208 through YvNorms._norm_forward
// :964-1007, whose CUDA path is the fused kernel of opss/kernels/fused_rms_norm.py): per row,
// acc = Σ x² in fp32, rms = sqrt(acc / H + eps), y = (x / rms) * w in fp32, rounded once to
// the activation dtype; with a bias, y + b rounded again (the bias is added to the kernel's
// output, norms.py:998-999). x / rms is taken as x * (1 / rms), one fp32 rounding more than a
// division (the product is within one fp32 ulp of the quotient), which keeps the kernel at
// the HBM bound instead of the VALU bound of one IEEE division per element.
//
// Two wavefronts per row (four for batches under 2048 rows): 16-byte loads (8 bf16 / 4 fp32 per
// lane per step), the sum of squares in lane order then a DPP row-rotation reduction, the four
// DPP rows in order and the row's wavefronts in order, the row kept in registers between the
// passes (H <= 8192 bf16 / 4096 fp32; longer rows are read again). Two norms in sequence (the MoE input of YvHybridBlock is norm_mlp(norm_fusion(h)),
// model/core/hybrid.py:1359 and :1310) run in the same pass over the row.
#include <math.h>

#include "yvmoe_internal.h"

namespace yvmoe {
namespace {

typedef unsigned u32x4n __attribute__((ext_vector_type(4)));

template <int O>
__device__ __forceinline__ float ror16n(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), 0x120 + O, 0xf, 0xf, false));
}
__device__ __forceinline__ float wave_sum_n(float v) {
    v = v + ror16n<8>(v);
    v = v + ror16n<4>(v);
    v = v + ror16n<2>(v);
    v = v + ror16n<1>(v);
    auto at = [&](int l) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l)); };
    return ((at(0) + at(16)) + at(32)) + at(48);
}

typedef __bf16 bf16x2n __attribute__((ext_vector_type(2)));
typedef float f32x2n __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float bf16_lo(unsigned u) { return __uint_as_float(u << 16); }
__device__ __forceinline__ float bf16_hi(unsigned u) { return __uint_as_float(u & 0xffff0000u); }
// two fp32 values to a packed bf16 pair, round to nearest even (v_cvt_pk_bf16_f32)
__device__ __forceinline__ unsigned pack_bf16(float lo, float hi) {
    return __builtin_bit_cast(unsigned, __builtin_convertvector(f32x2n{lo, hi}, bf16x2n));
}

// ACT: activation dtype; NN: RMSNorms applied in sequence (1 or 2), each rounded to ACT before
// the next one reads it, as two YvRMSNorm modules called one after the other round; WPR:
// wavefronts per row (2: half a row's registers per wavefront, 60 → 49 us at 16,721 rows
// against 1; 4 for small batches so that the 256 CUs have rows to work on; 1 is supported).
// Thread r of a row (r < 64 WPR) owns the 16-byte chunks c = r + 64 WPR i.
template <int ACT, int NN, int WPR>
__global__ __launch_bounds__(256) void rmsnorm_kernel(const void* x, NormChain nc, int N, int H,
                                                      void* y) {
    constexpr int EPC = ACT == YVMOE_ACT_BF16 ? 8 : 4;  // elements per 16-byte chunk
    constexpr int TPR = 64 * WPR;                       // threads per row
    constexpr int MAXC = 16 / WPR;                      // chunks per thread held in registers
    constexpr int RPB = 256 / TPR;  // rows per work-group
    __shared__ float s_part[RPB][NN][4];
    const int r = threadIdx.x % TPR;
    const int slot = threadIdx.x / TPR;
    const int row_id = blockIdx.x * RPB + slot;
    if (WPR == 1 && row_id >= N) return;  // no barrier in a one-wavefront row
    // several wavefronts per row share barriers: a row past N computes on a copy of the last
    // row and stores nothing
    const bool live = row_id < N;
    const int row = live ? row_id : N - 1;
    const int nch = H / EPC;  // H % EPC == 0 (checked on the host)
    const size_t rb = (size_t)row * H * (ACT == YVMOE_ACT_BF16 ? 2 : 4);
    const u32x4n* xr = (const u32x4n*)((const char*)x + rb);
    u32x4n* yr = (u32x4n*)((char*)y + rb);

    auto sumsq = [](u32x4n t) {
        float a = 0.f;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (ACT == YVMOE_ACT_BF16) {
                const float lo = bf16_lo(t[q]), hi = bf16_hi(t[q]);
                a += lo * lo;
                a += hi * hi;
            } else {
                const float v = __uint_as_float(t[q]);
                a += v * v;
            }
        }
        return a;
    };
    // one norm applied to chunk c of the row: x * (1 / rms) * w rounded, then + b rounded
    auto norm_chunk = [&](u32x4n t, int c, float rinv, int n) {
        const u32x4n ww = ((const u32x4n*)nc.w[n])[c];
        u32x4n o;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (ACT == YVMOE_ACT_BF16)
                o[q] = pack_bf16((bf16_lo(t[q]) * rinv) * bf16_lo(ww[q]),
                                 (bf16_hi(t[q]) * rinv) * bf16_hi(ww[q]));
            else
                o[q] = __float_as_uint((__uint_as_float(t[q]) * rinv) * __uint_as_float(ww[q]));
        }
        if (nc.b[n] != nullptr) {
            const u32x4n bb = ((const u32x4n*)nc.b[n])[c];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                if (ACT == YVMOE_ACT_BF16)
                    o[q] = pack_bf16(bf16_lo(o[q]) + bf16_lo(bb[q]), bf16_hi(o[q]) + bf16_hi(bb[q]));
                else
                    o[q] = __float_as_uint(__uint_as_float(o[q]) + __uint_as_float(bb[q]));
            }
        }
        return o;
    };
    // 1 / sqrt(Σx²/H + eps): wavefront sums, then the row's wavefronts in order
    auto rinv_of = [&](float acc, int n) {
        float tot = wave_sum_n(acc);
        if (WPR > 1) {
            if ((threadIdx.x & 63) == 0) s_part[slot][n][r >> 6] = tot;
            __syncthreads();
            tot = s_part[slot][n][0];
#pragma unroll
            for (int w = 1; w < WPR; ++w) tot += s_part[slot][n][w];
        }
        return 1.0f / sqrtf(tot / (float)H + nc.eps[n]);
    };

    if (nch <= TPR * MAXC) {
        // the row stays in registers: one read of x, one write of y
        u32x4n v[MAXC];
        float acc = 0.f;
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            const int c = r + TPR * i;
            v[i] = c < nch ? xr[c] : u32x4n{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int i = 0; i < MAXC; ++i) acc += sumsq(v[i]);
#pragma unroll
        for (int n = 0; n < NN - 1; ++n) {
            const float rinv = rinv_of(acc, n);
            acc = 0.f;
#pragma unroll
            for (int i = 0; i < MAXC; ++i) {
                const int c = r + TPR * i;
                if (c < nch) {
                    v[i] = norm_chunk(v[i], c, rinv, n);
                    acc += sumsq(v[i]);
                }
            }
        }
        const float rinv = rinv_of(acc, NN - 1);
#pragma unroll
        for (int i = 0; i < MAXC; ++i) {
            const int c = r + TPR * i;
            if (live && c < nch) yr[c] = norm_chunk(v[i], c, rinv, NN - 1);
        }
    } else {
        // long rows: the intermediate norm goes through y (each thread re-reads only the
        // chunks it wrote itself)
        float acc = 0.f;
        for (int c = r; c < nch; c += TPR) acc += sumsq(xr[c]);
        const u32x4n* src = xr;
        for (int n = 0; n < NN - 1; ++n) {
            const float rinv = rinv_of(acc, n);
            acc = 0.f;
            for (int c = r; c < nch; c += TPR) {
                const u32x4n o = norm_chunk(src[c], c, rinv, n);
                if (live) yr[c] = o;
                acc += sumsq(o);
            }
            src = yr;
        }
        const float rinv = rinv_of(acc, NN - 1);
        if (live)
            for (int c = r; c < nch; c += TPR) yr[c] = norm_chunk(src[c], c, rinv, NN - 1);
    }
}

}  // namespace

template <int ACT, int NN>
void rmsnorm_dispatch(const void* x, const NormChain& nc, int N, int H, void* y, hipStream_t st) {
    // two wavefronts per row once the rows fill the chip; four per row below that
    if (N >= 2048)
        rmsnorm_kernel<ACT, NN, 2><<<(unsigned)((N + 1) / 2), 256, 0, st>>>(x, nc, N, H, y);
    else
        rmsnorm_kernel<ACT, NN, 4><<<(unsigned)N, 256, 0, st>>>(x, nc, N, H, y);
}

int rmsnorm_launch(const void* x, int act, int N, int H, const NormChain& nc, int nn, void* y,
                   hipStream_t st) {
    if (N <= 0) return YVMOE_OK;
    if (act == YVMOE_ACT_BF16) {
        if (nn == 1) rmsnorm_dispatch<YVMOE_ACT_BF16, 1>(x, nc, N, H, y, st);
        else rmsnorm_dispatch<YVMOE_ACT_BF16, 2>(x, nc, N, H, y, st);
    } else {
        if (nn == 1) rmsnorm_dispatch<YVMOE_ACT_F32, 1>(x, nc, N, H, y, st);
        else rmsnorm_dispatch<YVMOE_ACT_F32, 2>(x, nc, N, H, y, st);
    }
    YV_LAUNCH_CHECK("rmsnorm");
    return YVMOE_OK;
}

}  // namespace yvmoe
