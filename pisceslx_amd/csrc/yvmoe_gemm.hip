// Expert GEMMs, router GEMM and combine of the Yv MoE layer for gfx950 (CDNA4).
//
// Reference: PiscesLxFusedMoEDispatch.forward opss/infer/fused_moe.py:54-123 (per-expert
// loop and index_add_ combine), YvSwiGLUExpert.forward model/moe/expert.py:475-489,
// YvDynamicMoELayer._compute_shared_expert_output model/moe/layer.py:812-865, the gate
// projection model/moe/gate.py:1179 and the complexity predictor gate.py:1112-1117.
//
// Tiling. A work-group is 4 wavefronts. It owns one 64-row tile of one expert segment
// (rows are expert-sorted slots; shared experts are extra segments of all N tokens) and
// 4 * NCB * 16 output columns; each wavefront owns NCB 16-column blocks over the whole K
// range and up to four 16-row MFMA blocks (only the row blocks that hold rows are
// computed). The B operand (weights, [out][in] row-major as nn.Linear stores them) streams
// from HBM with 16-byte loads per lane and is dequantized in registers to bf16; the A
// operand (activations gathered through the permutation) comes through L1/L2.
//
// Rounding points follow the reference's bf16 path, because the reference's own bf16
// chain sits about 2e-2 (max-abs) from exact arithmetic at these shapes and a more exact
// chain would not stay within that distance of it: weights are dequantized to
// bf16(q * s) before the product (the reference dequantizes, then runs F.linear in bf16);
// gate and up outputs, silu(gate), the product h and the down output are each rounded to
// bf16 (YvSwiGLUExpert.forward, model/moe/expert.py:484-489). Products accumulate in fp32.
// MFMA: v_mfma_f32_16x16x32_bf16 for bf16 activations, v_mfma_f32_16x16x4_f32 for fp32.
// Lane l holds A[row l%16][k-chunk l/16] and B[k-chunk l/16][col l%16]; the accumulator
// holds D[row 4*(l/16)+i][col l%16]. Each lane loads 16 consecutive k (bf16 path) or 4
// (fp32 path); the two (four) MFMAs of a k-step use the same k permutation for A and B,
// which leaves the sum unchanged.
#include <algorithm>

#include <type_traits>

#include "yvmoe_internal.h"

#ifndef YV_NB1
#define YV_NB1 1  // column blocks per wavefront, streaming gate/up (1 measured best)
#endif
#ifndef YV_NB2
#define YV_NB2 1  // column blocks per wavefront, streaming down projection (1 measured best)
#endif
#ifndef YV_DPF
#define YV_DPF true  // dense streaming with 64-row tiles: weights one chunk ahead
#endif
#ifndef YV_U1
#define YV_U1 4  // k-steps per staged chunk, streaming gate/up
#endif
#ifndef YV_PF1
#define YV_PF1 false  // streaming gate/up: weights one chunk ahead (false measured best)
#endif
#ifndef YV_WV1
#define YV_WV1 4  // wavefronts per work-group, streaming gate/up (4 measured best)
#endif
#ifndef YV_WV2
#define YV_WV2 4  // wavefronts per work-group, streaming down projection (4 measured best)
#endif
#ifndef YV_PF2
#define YV_PF2 false  // streaming down projection: weights one chunk ahead (false measured best)
#endif
#ifndef YV_U2
#define YV_U2 4  // k-steps per staged chunk, streaming down projection
#endif
#ifndef YV_PTILE
// persistent 8-wavefront int8 tile form (the next item's first chunks loaded during the current
// item's last chunk and epilogue): 0 off, 1 down projection only, 2 both projections. cfg3 FFN on
// alternating runs, same bits: 2 -1.0 / -1.3 / -1.4 %; 1 and gate/up alone ±0
#define YV_PTILE 2
#endif
#ifndef YV_PFP8
// fp8 on the persistent 8-wavefront form (block scales from a per-item LDS table): cfg5 FFN
// 6.86-6.87 -> 6.99 ms on alternating runs, same bits; off
#define YV_PFP8 0
#endif

namespace yvmoe {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef unsigned u32x4 __attribute__((ext_vector_type(4)));  // staging registers (plain vector)
typedef unsigned u32x2 __attribute__((ext_vector_type(2)));

// Weight loads of the streaming kernel: at decode sizes every weight byte is read by one
// work-group (a few for the shared experts, right after each other), so the loads are
// non-temporal — they do not push the activation rows, which every work-group of a tile
// reads again, out of L2.
__device__ __forceinline__ uint4 nt_load16(const char* p) {
    const u32x4 v = __builtin_nontemporal_load((const u32x4*)p);
    return make_uint4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ uint2 nt_load8(const char* p) {
    const u32x2 v = __builtin_nontemporal_load((const u32x2*)p);
    return make_uint2(v.x, v.y);
}

enum Epi { EPI_F32 = 0, EPI_SWIGLU = 1, EPI_DOWN = 2 };

struct GemmParams {
    const void* A;
    int lda;
    const int* rowmap;  // sorted row -> flat slot (the routing's perm); nullptr: A row = row
    int rowdiv;         // slots per token: token of a routed row = rowmap[row] / rowdiv
    int routed_rows;    // rows >= routed_rows are shared rows (token = (row - routed) % ntok)
    int ntok;
    const void* B0;
    const void* B1;
    const void* S0;
    const void* S1;
    long long b_stride;  // per expert, in weight elements (int4: codes, two per byte)
    long long s_stride;  // per expert, in scale elements
    int K;
    int ncols;
    void* out;
    int ldo;
    const int* tile_seg;
    const int* tile_row0;
    const int* ntiles;
    const int* seg_start;
    int nrows;  // rows when there is no tile table
    int kchunk;              // K range of one split (multiple of 64); K when not split
    long long split_stride;  // output elements between splits (EPI_F32 partial sums)
    const float* col_bias;   // EPI_F32: added to columns < col_bias_n by split 0 (or NULL)
    int col_bias_n;
    int nshared;             // shared experts (their tiles end the table; streaming WS form)
};

// EPI_F32 output value of column n for split kz: the accumulator plus the column bias.
__device__ __forceinline__ float f32_out(const GemmParams& p, float acc, int n, int kz) {
    return (p.col_bias != nullptr && kz == 0 && n < p.col_bias_n) ? acc + p.col_bias[n] : acc;
}

// Round-to-nearest-even fp32 -> bf16 pair (v_cvt_pk_bf16_f32), lo in bits 0..15.
__device__ __forceinline__ unsigned pack_bf16(float lo, float hi) {
    const bf16x2 v = __builtin_convertvector(f32x2{lo, hi}, bf16x2);
    return __builtin_bit_cast(unsigned, v);
}
__device__ __forceinline__ unsigned short f32_to_bf16_rne(float f) {
    return (unsigned short)(pack_bf16(f, 0.0f) & 0xffffu);
}
__device__ __forceinline__ float bf16_to_f32(unsigned short h) {
    return __uint_as_float((unsigned)h << 16);
}
__device__ __forceinline__ float round_bf16(float f) { return bf16_to_f32(f32_to_bf16_rne(f)); }
// The two fp16 halves of a register, widened (folded into a v_fma_mix_f32 operand select).
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ float f16_lo(unsigned v) { return (float)__builtin_bit_cast(f16x2, v).x; }
__device__ __forceinline__ float f16_hi(unsigned v) { return (float)__builtin_bit_cast(f16x2, v).y; }

union Frag16 {  // 16 bf16 = two MFMA operands
    uint4 u[2];
    bf16x8 v[2];
};

// -------------------------------------------------------------- B fragment loaders
// Each loads the 16 k-values of one output column for this lane's k-chunk and returns
// them as two bf16x8 operands holding bf16(q * s) (the reference's dequantized weights).
template <int WF>
struct BLoad;

// Weight operands (expert matrices, the router and gate projections; all but fp32) are stored
// in 16-row x 64-column blocks (pisceslx_amd/quant.py block_matrix): lane l = 16 g + r of a
// 16-column group reads piece (g, r) of each block, a contiguous 16 bytes per lane (8 for
// int4; bf16 pieces are split in two halves 1 KB apart). bptr() is the lane's address of its
// piece in the first block of column group n / 16 from K offset kbeg; load_blk() reads the
// piece of the ks-th 64-wide block after it (load_blk_nt() non-temporally); ptr() / load()
// address the row-major order.
template <>
struct BLoad<YVMOE_W_BF16> {
    typedef Frag16 Raw;
    static constexpr int BLK = 2048;
    static __device__ __forceinline__ const char* bptr(const void* base, long long e_off, int n,
                                                       int K, int kbeg, int lane) {
        return (const char*)base + e_off * 2 + ((long long)(n >> 4) * (K / 64) + kbeg / 64) * BLK +
               lane * 16;
    }
    static __device__ __forceinline__ void load_blk(Raw& r, const char* p, int ks) {
        r.u[0] = *(const uint4*)(p + (size_t)ks * BLK);
        r.u[1] = *(const uint4*)(p + (size_t)ks * BLK + 1024);
    }
    static __device__ __forceinline__ void load_blk_nt(Raw& r, const char* p, int ks) {
        r.u[0] = nt_load16(p + (size_t)ks * BLK);
        r.u[1] = nt_load16(p + (size_t)ks * BLK + 1024);
    }
    static __device__ __forceinline__ void cvt(const Raw& r, float, Frag16& f) { f = r; }
};

template <>
struct BLoad<YVMOE_W_INT8> {
    typedef uint4 Raw;
    static constexpr int BLK = 1024;
    static __device__ __forceinline__ const char* bptr(const void* base, long long e_off, int n,
                                                       int K, int kbeg, int lane) {
        return (const char*)base + e_off + ((long long)(n >> 4) * (K / 64) + kbeg / 64) * BLK + lane * 16;
    }
    static __device__ __forceinline__ void load_blk(Raw& r, const char* p, int ks) {
        r = *(const uint4*)(p + (size_t)ks * BLK);
    }
    static __device__ __forceinline__ void load_blk_nt(Raw& r, const char* p, int ks) {
        r = nt_load16(p + (size_t)ks * BLK);
    }
    static __device__ __forceinline__ void cvt(const Raw& r, float s, Frag16& f) {
        const unsigned w[4] = {r.x, r.y, r.z, r.w};
        unsigned o[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const float a = (float)(int)(signed char)(w[i] & 0xffu);
            const float b = (float)(int)(signed char)((w[i] >> 8) & 0xffu);
            const float c = (float)(int)(signed char)((w[i] >> 16) & 0xffu);
            const float d = (float)((int)w[i] >> 24);
            o[2 * i] = pack_bf16(a * s, b * s);
            o[2 * i + 1] = pack_bf16(c * s, d * s);
        }
        f.u[0] = make_uint4(o[0], o[1], o[2], o[3]);
        f.u[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
};

template <>
struct BLoad<YVMOE_W_INT4> {
    typedef uint2 Raw;
    static constexpr int BLK = 512;
    static __device__ __forceinline__ const char* bptr(const void* base, long long e_off, int n,
                                                       int K, int kbeg, int lane) {
        return (const char*)base + e_off / 2 + ((long long)(n >> 4) * (K / 64) + kbeg / 64) * BLK + lane * 8;
    }
    static __device__ __forceinline__ void load_blk(Raw& r, const char* p, int ks) {
        r = *(const uint2*)(p + (size_t)ks * BLK);
    }
    static __device__ __forceinline__ void load_blk_nt(Raw& r, const char* p, int ks) {
        r = nt_load8(p + (size_t)ks * BLK);
    }
    // bf16((q - 8) * s) for the 16 nibbles q (byte j: k = 2j low nibble, 2j + 1 high): one
    // and-or per two nibbles builds two fp16 values, 1024 + q for nibbles at bits 0-3 / 16-19
    // of a word (or of the word shifted by 8) and 1024 + 16 q for those at bits 4-7 / 20-23,
    // and one fused multiply-add of mixed precision (v_fma_mix_f32) gives
    // (1024 + q) * s - 1032 * s, or (1024 + 16 q) * (s / 16) - 72 * s, = (q - 8) * s with a
    // single rounding of an exact value (every term fits in 24 bits), which the pack rounds to
    // bf16 — the same bits as converting q - 8 and multiplying (checked on every bf16 scale
    // 2^-126 <= |s| < 2^97 and every nibble in every position; q = 8 with a negative scale gives
    // +0 instead of -0). About 2.3 VALU instructions per weight instead of 3.9.
    static __device__ __forceinline__ void cvt(const Raw& r, float s, Frag16& f) {
        const unsigned w[2] = {r.x, r.y};
        const float c0 = -1032.0f * s, s16 = s * 0.0625f, c1 = -72.0f * s;
        unsigned o[8];
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const unsigned w8 = w[i] >> 8;
            const unsigned a = (w[i] & 0x000F000Fu) | 0x64006400u;  // k 0, 4 (1024 + q)
            const unsigned b = (w[i] & 0x00F000F0u) | 0x64006400u;  // k 1, 5 (1024 + 16 q)
            const unsigned c = (w8 & 0x000F000Fu) | 0x64006400u;    // k 2, 6
            const unsigned d = (w8 & 0x00F000F0u) | 0x64006400u;    // k 3, 7
            o[4 * i + 0] = pack_bf16(__builtin_fmaf(f16_lo(a), s, c0), __builtin_fmaf(f16_lo(b), s16, c1));
            o[4 * i + 1] = pack_bf16(__builtin_fmaf(f16_lo(c), s, c0), __builtin_fmaf(f16_lo(d), s16, c1));
            o[4 * i + 2] = pack_bf16(__builtin_fmaf(f16_hi(a), s, c0), __builtin_fmaf(f16_hi(b), s16, c1));
            o[4 * i + 3] = pack_bf16(__builtin_fmaf(f16_hi(c), s, c0), __builtin_fmaf(f16_hi(d), s16, c1));
        }
        f.u[0] = make_uint4(o[0], o[1], o[2], o[3]);
        f.u[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
};

template <>
struct BLoad<YVMOE_W_FP8> {
    typedef uint4 Raw;
    static constexpr int BLK = 1024;
    static __device__ __forceinline__ const char* bptr(const void* base, long long e_off, int n,
                                                       int K, int kbeg, int lane) {
        return (const char*)base + e_off + ((long long)(n >> 4) * (K / 64) + kbeg / 64) * BLK + lane * 16;
    }
    static __device__ __forceinline__ void load_blk(Raw& r, const char* p, int ks) {
        r = *(const uint4*)(p + (size_t)ks * BLK);
    }
    static __device__ __forceinline__ void load_blk_nt(Raw& r, const char* p, int ks) {
        r = nt_load16(p + (size_t)ks * BLK);
    }
    static __device__ __forceinline__ void cvt(const Raw& r, float s, Frag16& f) {
        const unsigned w[4] = {r.x, r.y, r.z, r.w};
        unsigned o[8];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            // e4m3fn -> f32 is exact; q * s is rounded in fp32, then to bf16 (as the reference's
            // fp32 dequant followed by the cast to bf16)
            const f32x2 a = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], false);
            const f32x2 b = __builtin_amdgcn_cvt_pk_f32_fp8((int)w[i], true);
            o[2 * i] = pack_bf16(a.x * s, a.y * s);
            o[2 * i + 1] = pack_bf16(b.x * s, b.y * s);
        }
        f.u[0] = make_uint4(o[0], o[1], o[2], o[3]);
        f.u[1] = make_uint4(o[4], o[5], o[6], o[7]);
    }
};

__device__ __forceinline__ int map_row(const GemmParams& p, int row) {
    if (p.rowmap == nullptr) return row;
    if (row < p.routed_rows) return p.rowmap[row] / p.rowdiv;
    return (row - p.routed_rows) % p.ntok;
}

__device__ __forceinline__ float silu(float g) { return g / (1.0f + expf(-g)); }

// Dequant scale of column n for the k-step starting at k0: int8 bf16 [n]; int4 bf16
// [n][K/128]; fp8 fp32 [n/128][K/128]; 1 for unscaled formats.
template <int WF>
__device__ __forceinline__ float b_scale(const void* S, long long e_off, int n, int K, int k0) {
    if constexpr (WF == YVMOE_W_INT8) {
        return bf16_to_f32(((const unsigned short*)S)[e_off + n]);
    } else if constexpr (WF == YVMOE_W_INT4) {
        return bf16_to_f32(((const unsigned short*)S)[e_off + (long long)n * (K / 128) + k0 / 128]);
    } else if constexpr (WF == YVMOE_W_FP8) {
        return ((const float*)S)[e_off + (long long)(n / 128) * (K / 128) + k0 / 128];
    } else {
        return 1.0f;
    }
}

template <int EPI>
struct NMat {
    static constexpr int value = (EPI == EPI_SWIGLU) ? 2 : 1;
};

// ------------------------------------------------------------------ bf16 activations
// RB: B-operand ring depth (weight loads run RB-1 k-steps ahead of the MFMAs); RA: A-operand
// ring depth (RA divides RB).
template <int WF, int EPI, int NCB, int MAXRB, int RB = 4, int RA = 2>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(GemmParams p) {
    constexpr int NM = NMat<EPI>::value;
    constexpr bool GROUPED = (WF == YVMOE_W_INT4 || WF == YVMOE_W_FP8);
    static_assert(RB % RA == 0, "A ring depth must divide the B ring depth");
    constexpr int R = RB;
    typedef BLoad<WF> BL;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int e = 0, row0, seg_end;
    if (p.tile_seg != nullptr) {
        const int tile = blockIdx.x;
        if (tile >= *p.ntiles) return;
        e = p.tile_seg[tile];
        row0 = p.tile_row0[tile];
        seg_end = p.seg_start[e + 1];
    } else {
        row0 = blockIdx.x * MAXRB * 16;
        if (row0 >= p.nrows) return;
        seg_end = p.nrows;
    }
    const int col0 = (blockIdx.y * 4 + wave) * NCB * 16;
    if (col0 >= p.ncols) return;
    const int nrb = min(MAXRB, (seg_end - row0 + 15) / 16);
    const int kl = (lane >> 4) * 16;  // this lane's k offset inside a 64-wide k-step
    const int kbeg = blockIdx.z * p.kchunk;
    const int nks = (min(p.K, kbeg + p.kchunk) - kbeg) / 64;

    const char* arow[MAXRB];
#pragma unroll
    for (int rb = 0; rb < MAXRB; ++rb) {
        int r = row0 + rb * 16 + (lane & 15);
        if (r >= seg_end) r = row0;
        arow[rb] = (const char*)p.A + ((long long)map_row(p, r) * p.lda + kbeg + kl) * 2;
    }
    const long long e_off = (long long)e * p.b_stride;
    const long long s_off = (long long)e * p.s_stride;
    const char* bptr[NM][NCB];
    const void* sptr[2] = {p.S0, p.S1};
    int ncol[NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
        ncol[cb] = col0 + cb * 16 + (lane & 15);
        bptr[0][cb] = BL::bptr(p.B0, e_off, ncol[cb], p.K, kbeg, lane);
        if constexpr (NM == 2) bptr[NM - 1][cb] = BL::bptr(p.B1, e_off, ncol[cb], p.K, kbeg, lane);
    }

    f32x4 acc[NM][NCB][MAXRB];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int rb = 0; rb < MAXRB; ++rb) acc[m][cb][rb] = f32x4{0.f, 0.f, 0.f, 0.f};

    typename BL::Raw braw[R][NM][NCB];
    // per-k-step scales for group-scaled formats (ring), one scale per column otherwise
    float sc[GROUPED ? R : 1][NM][NCB];
    if constexpr (!GROUPED) {
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) sc[0][m][cb] = b_scale<WF>(sptr[m], s_off, ncol[cb], p.K, 0);
    }
    auto load_b = [&](int slot_ks, typename BL::Raw (&dst)[NM][NCB], float (&sdst)[NM][NCB]) {
        const int k0 = slot_ks * 64;
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                BL::load_blk(dst[m][cb], bptr[m][cb], slot_ks);
                if constexpr (GROUPED)
                    sdst[m][cb] = b_scale<WF>(sptr[m], s_off, ncol[cb], p.K, kbeg + k0);
            }
    };
    // Loads are unconditional (k-step clamped to the last one, row blocks past nrb read the
    // tile's first row): with no branch around them the compiler can wait for exactly the
    // oldest in-flight load instead of draining the whole ring before every MFMA.
    auto load_a = [&](int ks, Frag16 (&af)[MAXRB]) {
#pragma unroll
        for (int rb = 0; rb < MAXRB; ++rb) {
            const uint4* q = (const uint4*)(arow[rb] + (size_t)ks * 128);
            af[rb].u[0] = q[0];
            af[rb].u[1] = q[1];
        }
    };
    auto mma = [&](const typename BL::Raw (&bw)[NM][NCB], const float (&bs)[NM][NCB],
                   const Frag16 (&af)[MAXRB]) {
#pragma unroll
        for (int m = 0; m < NM; ++m) {
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) {
                Frag16 bf;
                BL::cvt(bw[m][cb], bs[m][cb], bf);
#pragma unroll
                for (int rb = 0; rb < MAXRB; ++rb) {
                    if (rb < nrb) {
                        f32x4& dst = acc[m][cb][rb];
                        dst = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rb].v[0], bf.v[0], dst, 0, 0, 0);
                        dst = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rb].v[1], bf.v[1], dst, 0, 0, 0);
                    }
                }
            }
        }
    };
    auto kc = [&](int ks) { return ks < nks ? ks : nks - 1; };

    constexpr int SR = GROUPED ? R : 1;
    Frag16 abuf[RA][MAXRB];
    if (nks > 0) {
#pragma unroll
        for (int r = 0; r < RB - 1; ++r) load_b(kc(r), braw[r], sc[r % SR]);
#pragma unroll
        for (int r = 0; r < RA - 1; ++r) load_a(kc(r), abuf[r]);
    }
    int ks0 = 0;
    for (; ks0 + RB <= nks; ks0 += RB) {
#pragma unroll
        for (int r = 0; r < RB; ++r) {
            const int ks = ks0 + r;
            load_b(kc(ks + RB - 1), braw[(r + RB - 1) % RB], sc[((r + RB - 1) % RB) % SR]);
            load_a(kc(ks + RA - 1), abuf[(r + RA - 1) % RA]);
            mma(braw[r], sc[r % SR], abuf[r % RA]);
        }
    }
    // tail (fewer than RB steps): their weights are already in ring slots 0..nks-ks0-1
#pragma unroll
    for (int r = 0; r < RB - 1; ++r) {
        if (ks0 + r < nks) {
            load_a(kc(ks0 + r + RA - 1), abuf[(r + RA - 1) % RA]);
            mma(braw[r], sc[r % SR], abuf[r % RA]);
        }
    }

    // epilogue (bf16 rounding points of YvSwiGLUExpert.forward)
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
        const int n = ncol[cb];
#pragma unroll
        for (int rb = 0; rb < MAXRB; ++rb) {
            if (rb < nrb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = row0 + rb * 16 + (lane >> 4) * 4 + i;
                    if (r < seg_end) {
                        if constexpr (EPI == EPI_F32) {
                            ((float*)p.out)[blockIdx.z * p.split_stride + (long long)r * p.ldo + n] =
                                f32_out(p, acc[0][cb][rb][i], n, blockIdx.z);
                        } else if constexpr (EPI == EPI_SWIGLU) {
                            const float g = round_bf16(acc[0][cb][rb][i]);
                            const float u = round_bf16(acc[NM - 1][cb][rb][i]);
                            const float sg = round_bf16(silu(g));
                            ((unsigned short*)p.out)[(long long)r * p.ldo + n] = f32_to_bf16_rne(sg * u);
                        } else {
                            ((unsigned short*)p.out)[(long long)r * p.ldo + n] =
                                f32_to_bf16_rne(acc[0][cb][rb][i]);
                        }
                    }
                }
            }
        }
    }
}

// ------------------------------------------------------------------ bf16, streaming form
// Weight-streaming form for batches whose experts hold few rows (decode). A work-group of 4
// wavefronts owns one tile (up to 16*MAXRB rows of one expert); every wavefront streams one
// weight matrix over NB 16-column blocks: for the down projection 4 x NB blocks per
// work-group, for gate/up 2 x NB column blocks with a gate wavefront and an up wavefront each,
// which swap accumulators through LDS for the SwiGLU epilogue. The K loop runs in chunks of U
// k-steps: the work-group stages the chunk's activation rows once in LDS (double-buffered,
// rows padded by 16 bytes so the 16 row-lanes of a fragment read hit distinct banks), and
// each wavefront loads only its weights from HBM, in plain load-then-use batches (the pattern
// that measured closest to the HBM ceiling), reading activation fragments from LDS. More
// column blocks per wavefront put more weight bytes in flight per activation chunk and per
// barrier.
template <int WF, int EPI, int U, int MAXRB, int NB, bool PF = false, int WV = 4>
__device__ __forceinline__ void stream_item(const GemmParams& p, int tile, int cgroup, int kz,
                                            uint4 (&As)[2][16 * MAXRB * (U * 8 + 1)]) {
    constexpr bool SWIGLU = EPI == EPI_SWIGLU;
    constexpr bool GROUPED = (WF == YVMOE_W_INT4 || WF == YVMOE_W_FP8);
    constexpr int ROWS = 16 * MAXRB;
    constexpr int ROW_U4 = U * 8 + 1;            // uint4 per staged row (U*64 bf16 + pad)
    constexpr int CHUNK_U4 = ROWS * U * 8;       // uint4 of one chunk
    constexpr int NT = 64 * WV;                  // threads of the work-group (WV wavefronts)
    constexpr int PER_THREAD = CHUNK_U4 / NT;    // uint4 each thread stages per chunk
    static_assert(CHUNK_U4 % NT == 0, "chunk must split evenly over the work-group");
    static_assert(WV == 2 || WV == 4 || WV == 8, "two, four or eight wavefronts per work-group");
    static_assert(2 * ROWS * ROW_U4 * 16 >= (WV / 2) * 64 * MAXRB * NB * 16, "LDS too small for the swap");
    typedef BLoad<WF> BL;
    const int tid = threadIdx.x;
    const int lane = tid & 63;
    const int wave = tid >> 6;
    // grouped: tiles from the tile table; dense (no table): ROWS-row tiles of nrows rows
    const bool dense = p.tile_seg == nullptr;
    const int e = dense ? 0 : p.tile_seg[tile];
    const int row0 = dense ? tile * ROWS : p.tile_row0[tile];
    const int seg_end = dense ? p.nrows : p.seg_start[e + 1];
    const int nvalid = min(ROWS, seg_end - row0);
    const int nrb = (nvalid + 15) / 16;
    const int mat = SWIGLU ? (wave & 1) : 0;  // 0: gate (or down), 1: up
    // first column of block b of this wavefront
    const int colw = SWIGLU ? (cgroup * (WV / 2) + (wave >> 1)) * 16 * NB : (cgroup * WV + wave) * 16 * NB;
    // K range of split kz (EPI_F32 writes split kz's partial sums at kz * split_stride)
    const int kbeg = kz * p.kchunk;
    const int kend = min(p.K, kbeg + p.kchunk);
    const int nks = (kend - kbeg) / 64;
    const int nchunks = (nks + U - 1) / U;

    // staging: thread t copies uint4 q = t + j*NT of each chunk: row q / (U*8), column q % (U*8)
    const char* srow[PER_THREAD];
    int sdst[PER_THREAD], scol[PER_THREAD];
    bool sval[PER_THREAD];
#pragma unroll
    for (int j = 0; j < PER_THREAD; ++j) {
        const int q = tid + j * NT;
        const int r = q / (U * 8);
        scol[j] = q % (U * 8);
        sval[j] = r < nvalid;
        srow[j] = (const char*)p.A + (long long)map_row(p, row0 + (sval[j] ? r : 0)) * p.lda * 2;
        sdst[j] = r * ROW_U4 + scol[j];
    }
    auto stage_load = [&](int c, uint4 (&v)[PER_THREAD]) {
#pragma unroll
        for (int j = 0; j < PER_THREAD; ++j) {
            const int kk = kbeg + c * U * 64 + scol[j] * 8;  // element offset in the row
            v[j] = (sval[j] && kk < kend) ? *(const uint4*)(srow[j] + (size_t)kk * 2) : make_uint4(0, 0, 0, 0);
        }
    };
    auto stage_store = [&](int buf, const uint4 (&v)[PER_THREAD]) {
#pragma unroll
        for (int j = 0; j < PER_THREAD; ++j) As[buf][sdst[j]] = v[j];
    };

    const long long e_off = (long long)e * p.b_stride;
    const long long s_off = (long long)e * p.s_stride;
    const void* S = mat ? p.S1 : p.S0;
    bool active[NB];
    int n[NB];
    const char* bptr[NB];
    float scl[NB];
#pragma unroll
    for (int b = 0; b < NB; ++b) {
        const int c0 = colw + b * 16;
        active[b] = c0 < p.ncols;  // blocks past the last column still stage and sync
        n[b] = min(c0, p.ncols - 16) + (lane & 15);
        bptr[b] = BL::bptr(mat ? p.B1 : p.B0, e_off, n[b], p.K, kbeg, lane);
        scl[b] = b_scale<WF>(S, s_off, n[b], p.K, 0);
    }

    f32x4 acc[NB][MAXRB];
#pragma unroll
    for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int rb = 0; rb < MAXRB; ++rb) acc[b][rb] = f32x4{0.f, 0.f, 0.f, 0.f};

    // weights of chunk c (the tile's expert is all they depend on)
    typename BL::Raw bw[NB][U];
    float sg[NB][U];
    auto load_w = [&](int c) {
        const int ks0 = c * U;
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (active[b]) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int ks = min(ks0 + u, nks - 1);
                    BL::load_blk_nt(bw[b][u], bptr[b], ks);
                    if constexpr (GROUPED) sg[b][u] = b_scale<WF>(S, s_off, n[b], p.K, kbeg + ks * 64);
                    else sg[b][u] = scl[b];
                }
            }
        }
    };
    if constexpr (PF) {
        // Weights one chunk ahead in a second register set (for launches of few work-groups
        // per CU, whose weight bytes in flight would otherwise be one chunk per wavefront): the
        // loop is unrolled by two so the sets alternate without copies; every load and staging
        // step is unconditional (clamped to the last chunk, in bounds, never used), and the
        // MFMAs of k-steps past the end are skipped.
        typename BL::Raw bw2[NB][U];
        float sg2[NB][U];
        auto load_into = [&](int c, typename BL::Raw (&w)[NB][U], float (&sc)[NB][U]) {
            const int ks0 = c * U;
#pragma unroll
            for (int b = 0; b < NB; ++b) {
#pragma unroll
                for (int u = 0; u < U; ++u) {
                    const int ks = min(ks0 + u, nks - 1);
                    BL::load_blk_nt(w[b][u], bptr[b], ks);
                    if constexpr (GROUPED) sc[b][u] = b_scale<WF>(S, s_off, n[b], p.K, kbeg + ks * 64);
                    else sc[b][u] = scl[b];
                }
            }
        };
        auto body = [&](int c, typename BL::Raw (&cw)[NB][U], float (&cs)[NB][U],
                        typename BL::Raw (&nw)[NB][U], float (&ns)[NB][U]) {
            // the staging loads first: the wait for them before their LDS store (the counter
            // is in order) then leaves the next chunk's weights in flight
            uint4 nx[PER_THREAD];
            stage_load(min(c + 1, nchunks - 1), nx);
            load_into(min(c + 1, nchunks - 1), nw, ns);
            const uint4* arow = &As[c & 1][(lane & 15) * ROW_U4 + (lane >> 4) * 2];
#pragma unroll
            for (int u = 0; u < U; ++u) {
                if (c * U + u < nks) {
                    Frag16 af[MAXRB];
#pragma unroll
                    for (int rb = 0; rb < MAXRB; ++rb) {
                        af[rb].u[0] = arow[rb * 16 * ROW_U4 + u * 8];
                        af[rb].u[1] = arow[rb * 16 * ROW_U4 + u * 8 + 1];
                    }
#pragma unroll
                    for (int b = 0; b < NB; ++b) {
                        Frag16 bf;
                        BL::cvt(cw[b][u], cs[b][u], bf);
#pragma unroll
                        for (int rb = 0; rb < MAXRB; ++rb) {
                            if (rb < nrb) {
                                acc[b][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rb].v[0], bf.v[0], acc[b][rb], 0, 0, 0);
                                acc[b][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rb].v[1], bf.v[1], acc[b][rb], 0, 0, 0);
                            }
                        }
                    }
                }
            }
            stage_store((c + 1) & 1, nx);
            __syncthreads();
        };
        load_into(0, bw, sg);
        {
            uint4 v[PER_THREAD];
            stage_load(0, v);
            stage_store(0, v);
        }
        __syncthreads();
        for (int c = 0; c < nchunks; c += 2) {
            body(c, bw, sg, bw2, sg2);
            body(c + 1, bw2, sg2, bw, sg);
        }
    } else {
    // chunk 0's weight loads go out before the activation staging, which waits on the row map
    // and the activation loads: the first weights are in flight during that chain
    load_w(0);
    {
        uint4 v[PER_THREAD];
        stage_load(0, v);
        stage_store(0, v);
    }
    __syncthreads();
    for (int c = 0; c < nchunks; ++c) {
        const int ks0 = c * U;
        if (c > 0) load_w(c);
        uint4 nxt[PER_THREAD];
        if (c + 1 < nchunks) stage_load(c + 1, nxt);
        const uint4* arow = &As[c & 1][(lane & 15) * ROW_U4 + (lane >> 4) * 2];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (ks0 + u < nks) {
                Frag16 af[MAXRB];
#pragma unroll
                for (int rb = 0; rb < MAXRB; ++rb) {
                    if (rb < nrb) {
                        af[rb].u[0] = arow[rb * 16 * ROW_U4 + u * 8];
                        af[rb].u[1] = arow[rb * 16 * ROW_U4 + u * 8 + 1];
                    }
                }
#pragma unroll
                for (int b = 0; b < NB; ++b) {
                    if (active[b]) {
                        Frag16 bf;
                        BL::cvt(bw[b][u], sg[b][u], bf);
#pragma unroll
                        for (int rb = 0; rb < MAXRB; ++rb) {
                            if (rb < nrb) {
                                acc[b][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rb].v[0], bf.v[0], acc[b][rb], 0, 0, 0);
                                acc[b][rb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(af[rb].v[1], bf.v[1], acc[b][rb], 0, 0, 0);
                            }
                        }
                    }
                }
            }
        }
        if (c + 1 < nchunks) stage_store((c + 1) & 1, nxt);
        __syncthreads();
    }
    }

    if constexpr (SWIGLU) {
        // up wavefronts hand their accumulators to the gate wavefront of the same columns
        float* xchg = (float*)&As[0][0];
        auto xi = [&](int b, int rb, int i) { return ((((wave >> 1) * NB + b) * MAXRB + rb) * 4 + i) * 64 + lane; };
        if (mat == 1) {
#pragma unroll
            for (int b = 0; b < NB; ++b)
#pragma unroll
                for (int rb = 0; rb < MAXRB; ++rb)
#pragma unroll
                    for (int i = 0; i < 4; ++i) xchg[xi(b, rb, i)] = acc[b][rb][i];
        }
        __syncthreads();
        if (mat == 0) {
#pragma unroll
            for (int b = 0; b < NB; ++b) {
                if (!active[b]) continue;
#pragma unroll
                for (int rb = 0; rb < MAXRB; ++rb) {
                    if (rb < nrb) {
#pragma unroll
                        for (int i = 0; i < 4; ++i) {
                            const int r = row0 + rb * 16 + (lane >> 4) * 4 + i;
                            if (r < seg_end) {
                                const float g = round_bf16(acc[b][rb][i]);
                                const float u = round_bf16(xchg[xi(b, rb, i)]);
                                const float sgl = round_bf16(silu(g));
                                ((unsigned short*)p.out)[(long long)r * p.ldo + n[b]] = f32_to_bf16_rne(sgl * u);
                            }
                        }
                    }
                }
            }
        }
        __syncthreads();  // the exchange area is the next item's staging buffer
    } else {
#pragma unroll
        for (int b = 0; b < NB; ++b) {
            if (!active[b]) continue;
#pragma unroll
            for (int rb = 0; rb < MAXRB; ++rb) {
                if (rb < nrb) {
#pragma unroll
                    for (int i = 0; i < 4; ++i) {
                        const int r = row0 + rb * 16 + (lane >> 4) * 4 + i;
                        if (r < seg_end) {
                            if constexpr (EPI == EPI_F32)
                                ((float*)p.out)[kz * p.split_stride + (long long)r * p.ldo + n[b]] =
                                    f32_out(p, acc[b][rb][i], n[b], kz);
                            else
                                ((unsigned short*)p.out)[(long long)r * p.ldo + n[b]] = f32_to_bf16_rne(acc[b][rb][i]);
                        }
                    }
                }
            }
        }
    }
}

// One item of the ntiles x ngroups item space (tile fastest) per work-group. Consecutive
// work-group ids go to different XCDs (round-robin dispatch), so the item space is cut into 8
// contiguous ranges, one per XCD: the tiles that share weights (the 16-row tiles of a shared
// expert, which all read the same columns) then run together on one XCD and fetch those
// weights from HBM once into its L2 instead of once per tile.
//
// WS (16-row tiles only): the rows of shared experts (from routed_rows on, every token) run 64
// at a time on the 64-row form (one k-step per staged chunk, the next chunk's weights in
// flight: the same LDS as the 16-row form), so each shared weight is read and converted once
// per column group instead of once per 16-row tile. Those items take the first work-group ids
// and so start first: they are slower per item than the 16-row items (a barrier per k-step),
// and last in the launch they set its end (cfg2 decode layer step 214.4 -> 253.4 us when they
// kept their places among the tiles, 214.4 -> 207.5 us first; the same bits either way).
template <int WF, int EPI, int U, int MAXRB, int NB, bool PF = false, int WV = 4, bool WS = false>
__global__ __launch_bounds__(64 * WV) void gemm_stream_kernel(GemmParams p, int ngroups, int nsplit) {
    constexpr int A_N = 2 * 16 * MAXRB * (U * 8 + 1);
    constexpr int A_W = WS ? 2 * 64 * 9 : 0;
    __shared__ uint4 As_raw[A_N > A_W ? A_N : A_W];
    static_assert(!WS || MAXRB == 1, "wide shared rows beside 16-row tiles only");
    int nt = p.tile_seg == nullptr ? (p.nrows + 16 * MAXRB - 1) / (16 * MAXRB) : *p.ntiles;
    int b = blockIdx.x;
    if constexpr (WS) {
        // the first work-groups take the 64-row items of the shared experts (so they start
        // first), the rest the 16-row items of the routed tiles
        const int tps = (p.ntok + 15) / 16, lps = (p.ntok + 63) / 64;  // tiles, 64-row items per expert
        const int nlead = p.nshared * lps;
        const int nwide = nlead * ngroups * nsplit;
        nt -= p.nshared * tps;  // routed tiles
        if (b < nwide) {
            const int lead = b % nlead, rest = b / nlead;
            const int tile = nt + (lead / lps) * tps + (lead % lps) * 4;
            stream_item<WF, EPI, 1, 4, NB, true, WV>(p, tile, rest % ngroups, rest / ngroups,
                                                     *reinterpret_cast<uint4(*)[2][64 * 9]>(As_raw));
            return;
        }
        b -= nwide;
    }
    const int nitems = nt * ngroups * nsplit;
    const int per_xcd = (nitems + 7) / 8;
    const int local = b / 8;
    if (local >= per_xcd) return;
    const int item = (b % 8) * per_xcd + local;
    if (item >= nitems) return;
    const int rest = item / nt;  // tile fastest, then column group, then K split
    const int tile = item % nt;
    stream_item<WF, EPI, U, MAXRB, NB, PF, WV>(p, tile, rest % ngroups, rest / ngroups,
                                               *reinterpret_cast<uint4(*)[2][16 * MAXRB * (U * 8 + 1)]>(As_raw));
}

// ------------------------------------------------------------------ bf16, LDS-tiled form
// Tiled form for batches whose experts hold many rows (prefill). A work-group of 16
// wavefronts computes a 256-row x 256-column output tile over K in 64-wide chunks.
//
// Chunks travel HBM -> LDS by direct-to-LDS loads (global_load_lds_dwordx4: each lane names
// its own 16-byte source, the wavefront's 64 lanes fill 1 KB of LDS in lane order), two
// chunks ahead of the MFMAs through a 3-stage LDS ring, with no register staging: the
// activation rows are gathered through the permutation, the weights land as stored (1-byte
// codes or bf16). Wavefronts form a 2 x 8 grid: each owns 128 activation rows and 32 weight
// rows, reads its weight fragment once per chunk, dequantizes it to bf16(q * s) in registers
// and multiplies it against its 8 activation row blocks (16 wavefronts, about 120 VGPRs:
// 4 per SIMD). int8 weights without folded rows take a 1 x 8 grid of 8 wavefronts of 256 x
// 32 instead (about 200 VGPRs, 2 per SIMD): each weight is converted once per work-group, not
// twice, and each wavefront converts the next chunk's weights beside its MFMAs (below) —
// cfg3's FFN 1.3 % faster with the same bits; fp8 measured 1.7 % slower on it. For gate/up the
// weight tile is 128 gate rows then the 128 up rows of the same columns; wavefront w holds
// gate and up of columns 16 w .. 16 w + 15 and finishes SwiGLU in registers.
//
// Each lane's MFMA operands cover 16 consecutive k of the chunk (k group l / 16), split over
// the two MFMAs of a chunk in the same order for both operands. Activation rows (128 B) are
// swizzled in 16-byte chunks so the fragment reads run without bank conflicts (measured):
// chunk c of row r sits at c ^ (r & 7) ^ ((r >> 3) & 1), and lane L of a 1 KB direct load
// fetches the logical chunk that the swizzle places at position L. Weight blocks arrive in
// the order the fragment reads want (lane l reads bytes 16 l of its row block's 1 KB, and
// of the second 1 KB for bf16): contiguous, conflict-free, no swizzle.
constexpr int TBM = 256, TBN = 256, TBK = 64;
constexpr int TTHREADS = 1024;

typedef __attribute__((address_space(3))) void* lds_ptr_t;
typedef __attribute__((address_space(1))) void* gbl_ptr_t;

// Direct-to-LDS load of 16 bytes per lane: lane L's bytes land at dst + 16 L (dst is the
// same for the whole wavefront). The LDS base travels in M0, which the instruction reads:
// it is an input operand of the asm bound to M0 ("{m0}"), so the compiler writes M0 itself
// and knows its value, and the asm modifies no register the compiler reserves.
__device__ __forceinline__ void dma16(const void* src, void* dst) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_ptr_t)dst);
    asm volatile("global_load_lds_dwordx4 %0, off" : : "v"(src), "{m0}"(m0) : "memory");
}
// The same with 4 bytes per lane (256 B per wavefront at dst + 4 L).
__device__ __forceinline__ void dma4(const void* src, void* dst) {
    const unsigned m0 = __builtin_amdgcn_readfirstlane((unsigned)(size_t)(lds_ptr_t)dst);
    asm volatile("global_load_lds_dword %0, off" : : "v"(src), "{m0}"(m0) : "memory");
}

__device__ __forceinline__ int swz_a(int r, int c) {  // bytes, 128-byte rows
    return r * 128 + ((c ^ (r & 7) ^ ((r >> 3) & 1)) << 4);
}

// s_waitcnt immediate that waits for vmcnt <= n only (gfx9 encoding: vmcnt in bits 3:0 and
// 15:14, expcnt 6:4 and lgkmcnt 11:8 left at their maxima)
constexpr int vmcnt_only(int n) { return (n & 0xf) | ((n >> 4) << 14) | (0x7 << 4) | (0xf << 8); }

// FOLD: room for the kTileFold rows of a folded remainder. S4K: int4 only, the largest K whose
// group scales the LDS table holds (8192; with folded rows 5120 beside a 3-stage ring, 8192
// beside a 2-stage ring).
template <int WF, int S4K = 8192, bool FOLD = false, int NW = 16>
struct TileCfg {
    static constexpr bool I4 = WF == YVMOE_W_INT4;
    static constexpr int EB = (WF == YVMOE_W_BF16) ? 2 : 1;  // bytes per weight (int4: half)
    // LDS stages (160 KB of LDS)
    static constexpr int NST = (EB == 2 || (I4 && FOLD && S4K > 5120)) ? 2 : 3;
    // activation rows: the 256-row tile (and the rows a folded remainder adds)
    static constexpr int A_BYTES = (TBM + (FOLD ? kTileFold : 0)) * TBK * 2;
    static constexpr int B_BYTES = I4 ? TBN * TBK / 2 : TBN * TBK * EB;
    static constexpr int B_BLK = I4 ? 512 : 1024 * EB;  // bytes of a 16-row weight block
    // 1 KB direct loads per wavefront for the 256 rows; the 32 folded rows take one 256-byte
    // dword load per wavefront, issued only by tiles that hold such rows
    static constexpr int A_DMA = TBM * TBK * 2 / 1024 / NW;
    // weight direct loads per wavefront: 1 KB each (int4: 256 B dword loads, two per block)
    static constexpr int B_DMA = I4 ? 2 : B_BYTES / 1024 / NW;
    static constexpr int NPW = A_DMA + B_DMA;
    static constexpr int S4 = I4 ? TBN * (S4K / 128) : 1;  // int4: the tile's group scales
    // row blocks of 16 per wavefront: 16 wavefronts in a 2 x 8 grid own 128 rows each, 8 in a
    // 1 x 8 grid all 256 (1-byte codes without folding only)
    static constexpr int MBW = NW == 16 ? 8 : 16;
    static_assert(NW == 16 || (NW == 8 && !FOLD && !I4 && EB == 1), "8 wavefronts: 1-byte codes, no folding");
};
static_assert(kTileFold * TBK * 2 == 256 * (TTHREADS / 64), "one dword load per wavefront");

// Work items are (tile, column block) pairs, column block fastest, so the work-groups that
// run together share activation tiles and (mostly) one expert's weights. Consecutive
// work-group ids go to different XCDs (round-robin dispatch), so the item space is cut into 8
// contiguous ranges, one per XCD, to keep each XCD's L2 traffic on its own range.
// FOLD: the tile table folds remainders, so an expert's last tile may hold 256 + 1 .. kTileFold
// rows. Such a launch holds two copies of the tile loop and each work-group runs the one its
// tile needs: the copy without folded rows keeps the register use and schedule of a plain
// tile. Launches without folding (FOLD = false) carry only that copy.
template <int WF, int EPI, int S4K = 8192, bool FOLD = false, int NW = 16>
__global__ __launch_bounds__(64 * NW) void gemm_tile_kernel(GemmParams p, int ncb) {
    typedef TileCfg<WF, S4K, FOLD, NW> C;
    constexpr int MBW = C::MBW;
    constexpr bool SWIGLU = EPI == EPI_SWIGLU;
    constexpr bool WFIRST = WF != YVMOE_W_BF16;  // weights as the MFMA's first operand
    constexpr bool GROUPED = WF == YVMOE_W_FP8;
    constexpr long long B_CHUNK = C::B_BLK;  // bytes of a weight block (64-wide K step)
    __shared__ __attribute__((aligned(1024))) unsigned char lds_a[C::NST][C::A_BYTES];
    __shared__ __attribute__((aligned(1024))) unsigned char lds_b[C::NST][C::B_BYTES];
    __shared__ float lds_s[2][64];  // fp8: block scales of the tile's two 128-row weight blocks
    __shared__ unsigned short lds_s4[C::S4];  // int4: bf16 scale of tile row r, group q at r * K/128 + q
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wr = NW == 16 ? wave >> 3 : 0, wc = wave & 7;  // wavefront grid: rows x 32 weight rows
    // grouped: tiles from the tile table; dense (no table): 256-row tiles of nrows rows
    const bool dense = p.tile_seg == nullptr;
    const int ntl = dense ? (p.nrows + TBM - 1) / TBM : *p.ntiles;
    // fp32 output: the items also run over K splits (split kz: K range kz * kchunk .. + kchunk,
    // the last one shorter), column block fastest, then split, then tile
    const int nsplit = EPI == EPI_F32 ? (p.K + p.kchunk - 1) / p.kchunk : 1;
    const int total = ntl * ncb * nsplit;
    const int per_xcd = (total + 7) / 8;
    const int local = blockIdx.x / 8;
    if (local >= per_xcd) return;
    const int item = (blockIdx.x % 8) * per_xcd + local;
    if (item >= total) return;
    const int tile = item / (ncb * nsplit);
    const int kz = EPI == EPI_F32 ? (item / ncb) % nsplit : 0;
    const int cb = item % ncb;
    const int e = dense ? 0 : p.tile_seg[tile];
    const int row0 = dense ? tile * TBM : p.tile_row0[tile];
    const int seg_end = dense ? p.nrows : p.seg_start[e + 1];
    // output columns: gate/up -> 128 columns (x2 matrices); down -> 256 columns (fp32 output:
    // the last column block may end early, at ncols, a multiple of 16)
    const int n0 = SWIGLU ? cb * (TBN / 2) : cb * TBN;
    const int kbeg = EPI == EPI_F32 ? kz * p.kchunk : 0;
    const int nks = EPI == EPI_F32 ? (min(p.K, kbeg + p.kchunk) - kbeg) / TBK : p.K / TBK;
    const long long e_off = (long long)e * p.b_stride;
    const long long s_off = (long long)e * p.s_stride;

    // rows past the 256-row tile: an expert's last tile that holds a folded remainder
    // (1 .. kTileFold rows; a folding tile table leaves no larger gap to the next tile)
    const int ext = FOLD && !dense ? seg_end - row0 - TBM : 0;

    auto run_tile = [&](auto fold_tag) {
        constexpr bool XT = decltype(fold_tag)::value;

        // direct-load sources: activation block j of this wavefront holds tile rows 8 (A_DMA w + j)
        // .. + 7, lane L row + L / 8, logical chunk (L % 8) ^ (L / 8) ^ (block & 1)
        const char* a_src[C::A_DMA];
#pragma unroll
        for (int j = 0; j < C::A_DMA; ++j) {
            const int blk = wave * C::A_DMA + j;
            const int r = blk * 8 + lane / 8;
            const int lc = (lane % 8) ^ (lane / 8) ^ (blk & 1);
            const int gr = (row0 + r < seg_end) ? row0 + r : row0;
            a_src[j] = (const char*)p.A + ((long long)map_row(p, gr) * p.lda + kbeg + lc * 8) * 2;
        }
        // folded rows: wavefront w loads rows 256 + 2 w and + 1, lane L dword L % 4 of physical
        // chunk (L % 32) / 4 of row 256 + 2 w + L / 32 (the same swizzle as the other rows)
        const char* x_src;
        {
            const int r = TBM + 2 * wave + lane / 32;
            const int lc = ((lane % 32) / 4) ^ (r & 7) ^ ((r >> 3) & 1);
            const int gr = (row0 + r < seg_end) ? row0 + r : row0;
            x_src = (const char*)p.A + ((long long)map_row(p, gr) * p.lda + lc * 8) * 2 + (lane % 4) * 4;
        }
        // weight blocks: 16-row x 64-column blocks (1 KB per 1-byte block, two 1 KB halves per
        // bf16 block) land in LDS as stored, block after block
        // (int4: 512-byte blocks, each loaded as two 256-byte halves by one wavefront)
        const char* b_src[C::B_DMA];
        int b_dst[C::B_DMA];
#pragma unroll
        for (int j = 0; j < C::B_DMA; ++j) {
            // 8 wavefronts: each loads the two weight blocks it converts itself (gate/up: its gate
            // and its up block), so its own load count says when they are in LDS
            const int blk = (NW == 8 && SWIGLU) ? j * 8 + wave : wave * C::B_DMA + j;
            const int rb = C::I4 ? wave : blk / C::EB;           // 16-row block of the tile
            const int half = C::I4 ? j : blk % C::EB;
            const int r16 = rb * 16;
            const void* B = (SWIGLU && r16 >= TBN / 2) ? p.B1 : p.B0;
            int nb16 = SWIGLU ? n0 + (r16 & (TBN / 2 - 1)) : n0 + r16;
            // fp32 output: blocks past ncols load the last block (their wavefront skips its
            // MFMAs and stores nothing)
            if (EPI == EPI_F32 && nb16 >= p.ncols) nb16 = p.ncols - 16;
            const long long e_bytes = C::I4 ? e_off / 2 : e_off * C::EB;
            b_src[j] = (const char*)B + e_bytes + (long long)(nb16 >> 4) * (p.K / 64) * B_CHUNK +
                       (long long)(kbeg / TBK) * B_CHUNK +
                       (C::I4 ? half * 256 + lane * 4 : half * 1024 + lane * 16);
            b_dst[j] = C::I4 ? rb * 512 + half * 256 : blk * 1024;
        }

        // Quantized weights (WFIRST) are the MFMA's first operand: lane l supplies weight row
        // brow[nb] as operand row i = l % 16 of fragment nb, and its accumulator ends with output
        // row c = l % 16 of the row block and the columns of operand rows 4 (l / 16) .. + 3.
        // Gate/up: fragment nb is rows wc 16 + i of the gate (0) or up (1) half, so a lane holds
        // gate and up of the same 4 columns. Down: the wavefront's 32 rows are dealt out in
        // groups of four, group q = i / 4 of fragment nb taking rows 8 q + 4 ((q / 2) ^ nb) + i % 4,
        // so that lane l holds the 8 consecutive columns 8 (l / 16) .. + 7 (fragment 0 first for
        // l < 32) and the epilogue writes 16 bytes per lane; the LDS reads of a fragment still
        // cover 16 distinct 16-byte bank groups per 16 lanes.
        // bf16 weights (and so the fp32-output form) are the second operand (fragment nb = rows
        // 16 nb + i; gate/up as above): back-to-back MFMAs then share their first operand (the
        // activation fragment), which measured 16-25 % faster where no dequantization runs
        // between them (same results); the accumulator holds rows 4 (l / 16) .. + 3 and column
        // l % 16, stored element by element.
        int brow[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
            const int i = lane & 15, q = i >> 2;
            if constexpr (SWIGLU) brow[nb] = nb * (TBN / 2) + wc * 16 + i;
            else if constexpr (!WFIRST) brow[nb] = wc * 32 + nb * 16 + i;
            else brow[nb] = wc * 32 + q * 8 + 4 * ((q >> 1) ^ nb) + (i & 3);
        }
        float cs[2] = {1.0f, 1.0f};  // int8: per-column scales
        int sblk[2] = {0, 0};        // fp8: which of the tile's two scale blocks
        if constexpr (WF == YVMOE_W_INT8) {
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int r = brow[nb];
                const void* S = (SWIGLU && r >= TBN / 2) ? p.S1 : p.S0;
                cs[nb] = b_scale<WF>(S, s_off, SWIGLU ? n0 + (r & (TBN / 2 - 1)) : n0 + r, p.K, 0);
            }
        }
        if constexpr (C::I4) {
            // the tile's group scales into LDS before any direct load is in flight
            const int kg = p.K / 128;
            for (int i = t; i < TBN * kg; i += 64 * NW) {
                const int r = i / kg, q = i % kg;
                const void* S = (SWIGLU && r >= TBN / 2) ? p.S1 : p.S0;
                const int n = SWIGLU ? n0 + (r & (TBN / 2 - 1)) : n0 + r;
                lds_s4[i] = ((const unsigned short*)S)[s_off + (long long)n * kg + q];
            }
            __syncthreads();
        }
        if constexpr (GROUPED) {
            const int kb = p.K / 128;
            if (t < 2 * kb) {
                const int b = t / kb, q = t % kb;
                const void* S = (SWIGLU && b == 1) ? p.S1 : p.S0;
                const int n = SWIGLU ? n0 : n0 + b * 128;
                lds_s[b][q] = b_scale<WF>(S, s_off, n, p.K, q * 128);
            }
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) sblk[nb] = brow[nb] / 128;
            __syncthreads();
        }

        f32x4 acc[MBW][2];
#pragma unroll
        for (int i = 0; i < MBW; ++i) acc[i][0] = acc[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};

        // LDS byte offsets of this lane's fragment reads (k group g = lane / 16)
        const int g = lane >> 4;
        const int a_rd0 = swz_a(wr * MBW * 16 + (lane & 15), 2 * g), a_rd1 = swz_a(wr * MBW * 16 + (lane & 15), 2 * g + 1);
        int b_rd0[2], b_rd1[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {  // piece (g, row % 16) of the row's block (+ 1 KB)
            b_rd0[nb] = (brow[nb] >> 4) * C::B_BLK + (16 * g + (brow[nb] & 15)) * (C::I4 ? 8 : 16);
            b_rd1[nb] = b_rd0[nb] + 1024;
        }

        // The direct loads are issued from inline assembly: the compiler's own form of them makes
        // it wait for every outstanding direct load before each LDS read, which would serialize
        // the prefetch. Completion is tracked here instead, with explicit vmcnt waits.
#define YV_TILE_ISSUE(CHUNK, ST)                                                                       \
        do {                                                                                               \
            _Pragma("unroll") for (int j = 0; j < C::A_DMA; ++j)                                           \
                dma16(a_src[j] + (size_t)(CHUNK) * TBK * 2, &lds_a[ST][(wave * C::A_DMA + j) * 1024]);     \
            if (XT) dma4(x_src + (size_t)(CHUNK) * TBK * 2, &lds_a[ST][TBM * TBK * 2 + wave * 256]);      \
            _Pragma("unroll") for (int j = 0; j < C::B_DMA; ++j) {                                         \
                if constexpr (C::I4) dma4(b_src[j] + (size_t)(CHUNK) * B_CHUNK, &lds_b[ST][b_dst[j]]);     \
                else dma16(b_src[j] + (size_t)(CHUNK) * B_CHUNK, &lds_b[ST][b_dst[j]]);                    \
            }                                                                                              \
        } while (0)

        // 16-row blocks of this wavefront's 128 rows that hold rows of the segment: an expert's
        // last tile skips the MFMAs of the blocks past its end (loads and barriers stay uniform)
        const int live_mb = min(MBW, max(0, (seg_end - (row0 + wr * MBW * 16) + 15) / 16));
        // fp32 output: a wavefront whose 32 columns lie past ncols skips every MFMA (a separate
        // flag: folding it into live_mb made the compiler spill 59 VGPRs of this kernel)
        const bool colive = EPI != EPI_F32 || n0 + wc * 32 < p.ncols;
        // folded rows: wavefront row wr computes row block 256 + 16 wr .. + 15 when it holds rows
        const bool xlive = XT && ext > 16 * wr;
        f32x4 accx[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
        const int xa_rd0 = swz_a(TBM + wr * 16 + (lane & 15), 2 * g);
        const int xa_rd1 = swz_a(TBM + wr * 16 + (lane & 15), 2 * g + 1);

        YV_TILE_ISSUE(0, 0);
        if (C::NST == 3 && nks > 1) YV_TILE_ISSUE(1, 1);
        int st = 0;
        // 8 wavefronts of 256 x 32: a wavefront converts chunk c + 1's weights in the middle of
        // chunk c, beside the MFMAs of its last 8 row blocks, as soon as its own loads of them
        // have landed (it loads exactly the blocks it converts), so no conversion stands between
        // a barrier and the next MFMA. One barrier per chunk, as in the 16-wavefront loop; the
        // same MFMAs in the same order per accumulator, so the same bits.
        if constexpr (NW == 8) {
            auto bconv = [&](const unsigned char* Bs, int cc, bf16x8 (&bq)[2][2]) {
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    const u32x4 raw = *(const u32x4*)(Bs + b_rd0[nb]);
                    const float sc = GROUPED ? lds_s[sblk[nb]][(cc * TBK) / 128] : cs[nb];
                    Frag16 f;
                    BLoad<WF>::cvt(make_uint4(raw.x, raw.y, raw.z, raw.w), sc, f);
                    bq[nb][0] = f.v[0];
                    bq[nb][1] = f.v[1];
                }
            };
            const int nlm = colive ? live_mb : 0;
            bf16x8 bcur[2][2], bnext[2][2];
            if (nks > 1) __builtin_amdgcn_s_waitcnt(vmcnt_only(C::NPW));
            else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
            bconv(lds_b[0], 0, bcur);
            auto mb_step = [&](const unsigned char* As, int mb) {
                const bf16x8 a0 = *(const bf16x8*)(As + a_rd0 + mb * 16 * 128);
                const bf16x8 a1 = *(const bf16x8*)(As + a_rd1 + mb * 16 * 128);
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bcur[nb][0], a0, acc[mb][nb], 0, 0, 0);
                    acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bcur[nb][1], a1, acc[mb][nb], 0, 0, 0);
                }
            };
            // NMB row blocks (8 or 16): an expert's last tile computes past its end (rows not
            // stored) - one branch per tile instead of one per row block, whose 16 conditional
            // blocks spilled registers
            auto chunk = [&](auto nmb) {
                constexpr int NMB = decltype(nmb)::value;
                for (int c = 0; c < nks; ++c) {
                    // every wavefront's loads of chunk c have landed (each waited for its own) and
                    // all reads of chunk c - 1 are done: its stage takes chunk c + 2
                    asm volatile("" ::: "memory");
                    __builtin_amdgcn_s_barrier();
                    asm volatile("" ::: "memory");
                    if (c + 2 < nks) {
                        int sn = st + 2;
                        if (sn >= 3) sn -= 3;
                        YV_TILE_ISSUE(c + 2, sn);
                    }
                    const unsigned char* As = lds_a[st];
#pragma unroll
                    for (int mb = 0; mb < NMB / 2; ++mb) mb_step(As, mb);
                    int sx = st + 1;
                    if (sx >= 3) sx -= 3;
                    const bool more = c + 1 < nks;
                    if (more) {
                        // this wavefront's loads of chunk c + 1 (its weight blocks among them)
                        if (c + 2 < nks) __builtin_amdgcn_s_waitcnt(vmcnt_only(C::NPW));
                        else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
                        asm volatile("" ::: "memory");
                    }
                    // chunk c + 1's weights (after the last chunk: its own stage again, unused)
                    bconv(lds_b[more ? sx : st], more ? c + 1 : c, bnext);
#pragma unroll
                    for (int mb = NMB / 2; mb < NMB; ++mb) mb_step(As, mb);
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        bcur[nb][0] = bnext[nb][0];
                        bcur[nb][1] = bnext[nb][1];
                    }
                    st = sx;
                }
            };
            if (nlm > 8) chunk(std::integral_constant<int, 16>{});
            else if (nlm > 0) chunk(std::integral_constant<int, 8>{});
            else chunk(std::integral_constant<int, 0>{});
        } else
        for (int c = 0; c < nks; ++c) {
            // this wavefront's loads of chunk c have landed (the next chunk's may be in flight) ...
            if (C::NST == 3 && c + 1 < nks) {
                if (XT) __builtin_amdgcn_s_waitcnt(vmcnt_only(C::NPW + 1));
                else __builtin_amdgcn_s_waitcnt(vmcnt_only(C::NPW));
            } else {
                __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
            }
            // ... and after the barrier every wavefront's have, and all reads of chunk c - 1 are
            // done, so its stage can take chunk c + NST - 1
            asm volatile("" ::: "memory");
            __builtin_amdgcn_s_barrier();
            asm volatile("" ::: "memory");
            if (c + C::NST - 1 < nks) {
                int sn = st + C::NST - 1;
                if (sn >= C::NST) sn -= C::NST;
                YV_TILE_ISSUE(c + C::NST - 1, sn);
            }
            const unsigned char* As = lds_a[st];
            const unsigned char* Bs = lds_b[st];
            // one chunk of MFMAs; PART: only the row blocks below seg_end (an expert's last tile);
            // EXT: plus the folded row block
            auto compute = [&](auto part, auto extra) {
                constexpr bool PART = decltype(part)::value;
                constexpr bool EXT = decltype(extra)::value;
                bf16x8 bq[2][2];
#pragma unroll
                for (int nb = 0; nb < 2; ++nb) {
                    if constexpr (C::I4) {
                        const u32x2 raw = *(const u32x2*)(Bs + b_rd0[nb]);
                        const float s = bf16_to_f32(lds_s4[brow[nb] * (p.K / 128) + (c * TBK) / 128]);
                        Frag16 f;
                        BLoad<WF>::cvt(make_uint2(raw.x, raw.y), s, f);
                        bq[nb][0] = f.v[0];
                        bq[nb][1] = f.v[1];
                    } else if constexpr (C::EB == 1) {
                        const u32x4 raw = *(const u32x4*)(Bs + b_rd0[nb]);
                        const float s = GROUPED ? lds_s[sblk[nb]][(c * TBK) / 128] : cs[nb];
                        Frag16 f;
                        BLoad<WF>::cvt(make_uint4(raw.x, raw.y, raw.z, raw.w), s, f);
                        bq[nb][0] = f.v[0];
                        bq[nb][1] = f.v[1];
                    } else {
                        bq[nb][0] = *(const bf16x8*)(Bs + b_rd0[nb]);
                        bq[nb][1] = *(const bf16x8*)(Bs + b_rd1[nb]);
                    }
                }
#pragma unroll
                for (int mb = 0; mb < MBW; ++mb) {
                    if (PART && mb >= live_mb) continue;
                    const bf16x8 a0 = *(const bf16x8*)(As + a_rd0 + mb * 16 * 128);
                    const bf16x8 a1 = *(const bf16x8*)(As + a_rd1 + mb * 16 * 128);
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        if constexpr (WFIRST) {
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bq[nb][0], a0, acc[mb][nb], 0, 0, 0);
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bq[nb][1], a1, acc[mb][nb], 0, 0, 0);
                        } else {
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bq[nb][0], acc[mb][nb], 0, 0, 0);
                            acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bq[nb][1], acc[mb][nb], 0, 0, 0);
                        }
                    }
                }
                if constexpr (EXT) {
                    const bf16x8 a0 = *(const bf16x8*)(As + xa_rd0);
                    const bf16x8 a1 = *(const bf16x8*)(As + xa_rd1);
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        if constexpr (WFIRST) {
                            accx[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bq[nb][0], a0, accx[nb], 0, 0, 0);
                            accx[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bq[nb][1], a1, accx[nb], 0, 0, 0);
                        } else {
                            accx[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a0, bq[nb][0], accx[nb], 0, 0, 0);
                            accx[nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a1, bq[nb][1], accx[nb], 0, 0, 0);
                        }
                    }
                }
            };
            if (xlive) compute(std::false_type{}, std::true_type{});
            else if (live_mb == MBW && colive) compute(std::false_type{}, std::false_type{});
            else if (live_mb > 0 && colive) compute(std::true_type{}, std::false_type{});
            if (++st == C::NST) st = 0;
        }
#undef YV_TILE_ISSUE

        // epilogue: row l % 16 of each 16-row block; gate/up 4 consecutive columns (8-byte
        // stores), down 8 (16-byte stores)
        // one 16-row block at row rb: WFIRST, lane row rb + l % 16; else rows rb + 4 (l / 16) + i
        auto store_block = [&](int rb, f32x4 c0, f32x4 c1) {
            if constexpr (!WFIRST) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = rb + 4 * g + i;
                    if (r >= seg_end) continue;
                    if constexpr (SWIGLU) {
                        const int n = n0 + wc * 16 + (lane & 15);
                        const float gt = round_bf16(c0[i]);
                        const float up = round_bf16(c1[i]);
                        ((unsigned short*)p.out)[(long long)r * p.ldo + n] =
                            f32_to_bf16_rne(round_bf16(silu(gt)) * up);
                    } else {
#pragma unroll
                        for (int nb = 0; nb < 2; ++nb) {
                            const int n = n0 + wc * 32 + nb * 16 + (lane & 15);
                            const float v = nb ? c1[i] : c0[i];
                            if constexpr (EPI == EPI_F32) {
                                if (n < p.ncols)
                                    ((float*)p.out)[kz * p.split_stride + (long long)r * p.ldo + n] =
                                        f32_out(p, v, n, kz);
                            } else
                                ((unsigned short*)p.out)[(long long)r * p.ldo + n] = f32_to_bf16_rne(v);
                        }
                    }
                }
                return;
            }
            const int r = rb + (lane & 15);
            if (r >= seg_end) return;
            if constexpr (SWIGLU) {
                const int n = n0 + wc * 16 + 4 * g;
                float hv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float gt = round_bf16(c0[i]);
                    const float up = round_bf16(c1[i]);
                    hv[i] = round_bf16(silu(gt)) * up;
                }
                *(uint2*)((unsigned short*)p.out + (long long)r * p.ldo + n) =
                    make_uint2(pack_bf16(hv[0], hv[1]), pack_bf16(hv[2], hv[3]));
            } else {
                const int n = n0 + wc * 32 + 8 * g;
                const f32x4 lo = g < 2 ? c0 : c1;
                const f32x4 hi = g < 2 ? c1 : c0;
                *(uint4*)((unsigned short*)p.out + (long long)r * p.ldo + n) =
                    make_uint4(pack_bf16(lo[0], lo[1]), pack_bf16(lo[2], lo[3]),
                               pack_bf16(hi[0], hi[1]), pack_bf16(hi[2], hi[3]));
            }
        };
#pragma unroll
        for (int mb = 0; mb < MBW; ++mb) store_block(row0 + wr * MBW * 16 + mb * 16, acc[mb][0], acc[mb][1]);
        if (xlive) store_block(row0 + TBM + wr * 16, accx[0], accx[1]);
    };
    if (FOLD && ext > 0 && ext <= kTileFold) run_tile(std::integral_constant<bool, FOLD>{});
    else run_tile(std::false_type{});
}

// Persistent form of the 8-wavefront tile kernel for 1-byte codes (int8; fp8 measured slower on
// it and stays on gemm_tile_kernel's 16 wavefronts), no folded rows, K of at least 3 chunks:
// one work-group per CU walks its XCD's range of (tile, column block) items with the stride of
// that XCD's work-groups, so the work-groups of an XCD still run neighbouring items together.
// After the barrier that opens an item's last chunk, the two ring stages that chunk does not
// use are free: they take the next item's chunks 0 and 1, which land during the last chunk's
// MFMAs and the epilogue instead of after a new work-group's start. The arithmetic per item is
// the 8-wavefront loop of gemm_tile_kernel (the same bits). The next item's first wait also
// covers the epilogue's stores (they count in the same counter as the loads).
template <int WF, int EPI>
__global__ __launch_bounds__(512) void gemm_tile_persist_kernel(GemmParams p, int ncb) {
    typedef TileCfg<WF, 8192, false, 8> C;
    static_assert(WF == YVMOE_W_INT8 || WF == YVMOE_W_FP8, "1-byte codes");
    constexpr int MBW = C::MBW;
    constexpr bool SWIGLU = EPI == EPI_SWIGLU;
    constexpr bool GROUPED = WF == YVMOE_W_FP8;
    constexpr long long B_CHUNK = C::B_BLK;
    __shared__ __attribute__((aligned(1024))) unsigned char lds_a[3][C::A_BYTES];
    __shared__ __attribute__((aligned(1024))) unsigned char lds_b[3][C::B_BYTES];
    // fp8: block scales of the item's two 128-row weight blocks, one table per item in turn
    __shared__ float lds_s[GROUPED ? 2 : 1][2][64];
    const int t = threadIdx.x;
    const int lane = t & 63;
    const int wave = t >> 6;
    const int wc = wave;
    const int total = *p.ntiles * ncb;
    const int per_xcd = (total + 7) / 8;
    const int xend = min(total, (int)(blockIdx.x % 8) * per_xcd + per_xcd);
    const int stride = gridDim.x / 8;
    int item = (blockIdx.x % 8) * per_xcd + blockIdx.x / 8;
    if (item >= xend) return;
    const int nks = p.K / TBK;

    // item-independent: weight block of each direct load, fragment rows and LDS read offsets
    int b_blk[C::B_DMA];
#pragma unroll
    for (int j = 0; j < C::B_DMA; ++j) b_blk[j] = SWIGLU ? j * 8 + wave : wave * C::B_DMA + j;
    int brow[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
        const int i = lane & 15, q = i >> 2;
        brow[nb] = SWIGLU ? nb * (TBN / 2) + wc * 16 + i : wc * 32 + q * 8 + 4 * ((q >> 1) ^ nb) + (i & 3);
    }
    const int g = lane >> 4;
    const int a_rd0 = swz_a(lane & 15, 2 * g), a_rd1 = swz_a(lane & 15, 2 * g + 1);
    int b_rd0[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) b_rd0[nb] = (brow[nb] >> 4) * C::B_BLK + (16 * g + (brow[nb] & 15)) * 16;

    int sblk[2];  // fp8: which of the item's two scale blocks each fragment's rows use
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) sblk[nb] = brow[nb] / 128;

    // one item's addressing: direct-load sources and the two per-column scales (int8) or the
    // index of its block-scale table (fp8)
    struct Item {
        int row0, seg_end, n0, sbuf;
        const char* a_src[C::A_DMA];
        const char* b_src[C::B_DMA];
        float cs[2];
    };
    auto setup = [&](int it, Item& I, int sbuf) {
        const int tile = it / ncb, cb = it % ncb;
        const int e = p.tile_seg[tile];
        I.row0 = p.tile_row0[tile];
        I.seg_end = p.seg_start[e + 1];
        I.n0 = SWIGLU ? cb * (TBN / 2) : cb * TBN;
        const long long e_off = (long long)e * p.b_stride;
        const long long s_off = (long long)e * p.s_stride;
#pragma unroll
        for (int j = 0; j < C::A_DMA; ++j) {
            const int blk = wave * C::A_DMA + j;
            const int r = blk * 8 + lane / 8;
            const int lc = (lane % 8) ^ (lane / 8) ^ (blk & 1);
            const int gr = (I.row0 + r < I.seg_end) ? I.row0 + r : I.row0;
            I.a_src[j] = (const char*)p.A + ((long long)map_row(p, gr) * p.lda + lc * 8) * 2;
        }
#pragma unroll
        for (int j = 0; j < C::B_DMA; ++j) {
            const int r16 = b_blk[j] * 16;
            const void* B = (SWIGLU && r16 >= TBN / 2) ? p.B1 : p.B0;
            const int nb16 = SWIGLU ? I.n0 + (r16 & (TBN / 2 - 1)) : I.n0 + r16;
            I.b_src[j] = (const char*)B + e_off + (long long)(nb16 >> 4) * (p.K / 64) * B_CHUNK + lane * 16;
        }
        I.sbuf = sbuf;
        if constexpr (GROUPED) {
            // written a whole item before its first reader (the current item's barriers
            // publish it); the table it replaces belonged to the item before the current one
            I.cs[0] = I.cs[1] = 1.0f;
            const int kb = p.K / 128;
            if (t < 2 * kb) {
                const int b = t / kb, q = t % kb;
                const void* S = (SWIGLU && b == 1) ? p.S1 : p.S0;
                lds_s[sbuf][b][q] = b_scale<WF>(S, s_off, SWIGLU ? I.n0 : I.n0 + b * 128, p.K, q * 128);
            }
        } else {
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const int r = brow[nb];
                const void* S = (SWIGLU && r >= TBN / 2) ? p.S1 : p.S0;
                I.cs[nb] = b_scale<WF>(S, s_off, SWIGLU ? I.n0 + (r & (TBN / 2 - 1)) : I.n0 + r, p.K, 0);
            }
        }
    };
    auto issue = [&](const Item& I, int chunk, int st) {
#pragma unroll
        for (int j = 0; j < C::A_DMA; ++j)
            dma16(I.a_src[j] + (size_t)chunk * TBK * 2, &lds_a[st][(wave * C::A_DMA + j) * 1024]);
#pragma unroll
        for (int j = 0; j < C::B_DMA; ++j) dma16(I.b_src[j] + (size_t)chunk * B_CHUNK, &lds_b[st][b_blk[j] * 1024]);
    };

    Item cur, nxt;
    setup(item, cur, 0);
    int st = 0;
    issue(cur, 0, 0);
    issue(cur, 1, 1);
    if constexpr (GROUPED) __syncthreads();  // the first item's scale table
    for (;;) {
        const int next = item + stride;
        const bool has_next = next < xend;
        if (has_next) setup(next, nxt, cur.sbuf ^ 1);
        f32x4 acc[MBW][2];
#pragma unroll
        for (int i = 0; i < MBW; ++i) acc[i][0] = acc[i][1] = f32x4{0.f, 0.f, 0.f, 0.f};
        auto bconv = [&](const unsigned char* Bs, int cc, bf16x8 (&bq)[2][2]) {
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                const u32x4 raw = *(const u32x4*)(Bs + b_rd0[nb]);
                const float sc = GROUPED ? lds_s[cur.sbuf][sblk[nb]][(cc * TBK) / 128] : cur.cs[nb];
                Frag16 f;
                BLoad<WF>::cvt(make_uint4(raw.x, raw.y, raw.z, raw.w), sc, f);
                bq[nb][0] = f.v[0];
                bq[nb][1] = f.v[1];
            }
        };
        const int live_mb = min(MBW, max(0, (cur.seg_end - cur.row0 + 15) / 16));
        bf16x8 bcur[2][2], bnext[2][2];
        // chunk 0 of this item has landed (chunk 1's loads, the younger ones, may be in flight)
        __builtin_amdgcn_s_waitcnt(vmcnt_only(C::NPW));
        bconv(lds_b[st], 0, bcur);
        auto mb_step = [&](const unsigned char* As, int mb) {
            const bf16x8 a0 = *(const bf16x8*)(As + a_rd0 + mb * 16 * 128);
            const bf16x8 a1 = *(const bf16x8*)(As + a_rd1 + mb * 16 * 128);
#pragma unroll
            for (int nb = 0; nb < 2; ++nb) {
                acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bcur[nb][0], a0, acc[mb][nb], 0, 0, 0);
                acc[mb][nb] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bcur[nb][1], a1, acc[mb][nb], 0, 0, 0);
            }
        };
        auto chunk = [&](auto nmb) {
            constexpr int NMB = decltype(nmb)::value;
            for (int c = 0; c < nks; ++c) {
                asm volatile("" ::: "memory");
                __builtin_amdgcn_s_barrier();
                asm volatile("" ::: "memory");
                int s1 = st + 1;
                if (s1 >= 3) s1 -= 3;
                int s2 = st + 2;
                if (s2 >= 3) s2 -= 3;
                if (c + 2 < nks) {
                    issue(cur, c + 2, s2);
                } else if (c + 1 == nks && has_next) {
                    // the stages of chunks c - 2 and c - 1 are free: the next item's chunks 0, 1
                    issue(nxt, 0, s1);
                    issue(nxt, 1, s2);
                }
                const unsigned char* As = lds_a[st];
#pragma unroll
                for (int mb = 0; mb < NMB / 2; ++mb) mb_step(As, mb);
                const bool more = c + 1 < nks;
                if (more) {
                    if (c + 2 < nks) __builtin_amdgcn_s_waitcnt(vmcnt_only(C::NPW));
                    else __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
                    asm volatile("" ::: "memory");
                    bconv(lds_b[s1], c + 1, bnext);
                }
#pragma unroll
                for (int mb = NMB / 2; mb < NMB; ++mb) mb_step(As, mb);
                if (more) {
#pragma unroll
                    for (int nb = 0; nb < 2; ++nb) {
                        bcur[nb][0] = bnext[nb][0];
                        bcur[nb][1] = bnext[nb][1];
                    }
                }
                st = s1;
            }
        };
        if (live_mb > 8) chunk(std::integral_constant<int, 16>{});
        else if (live_mb > 0) chunk(std::integral_constant<int, 8>{});
        else chunk(std::integral_constant<int, 0>{});

        // epilogue (gemm_tile_kernel's WFIRST store_block)
        const int seg_end = cur.seg_end, n0 = cur.n0;
        auto store_block = [&](int rb, f32x4 c0, f32x4 c1) {
            const int r = rb + (lane & 15);
            if (r >= seg_end) return;
            if constexpr (SWIGLU) {
                const int n = n0 + wc * 16 + 4 * g;
                float hv[4];
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const float gt = round_bf16(c0[i]);
                    const float up = round_bf16(c1[i]);
                    hv[i] = round_bf16(silu(gt)) * up;
                }
                *(uint2*)((unsigned short*)p.out + (long long)r * p.ldo + n) =
                    make_uint2(pack_bf16(hv[0], hv[1]), pack_bf16(hv[2], hv[3]));
            } else {
                const int n = n0 + wc * 32 + 8 * g;
                const f32x4 lo = g < 2 ? c0 : c1;
                const f32x4 hi = g < 2 ? c1 : c0;
                *(uint4*)((unsigned short*)p.out + (long long)r * p.ldo + n) =
                    make_uint4(pack_bf16(lo[0], lo[1]), pack_bf16(lo[2], lo[3]),
                               pack_bf16(hi[0], hi[1]), pack_bf16(hi[2], hi[3]));
            }
        };
#pragma unroll
        for (int mb = 0; mb < MBW; ++mb) store_block(cur.row0 + mb * 16, acc[mb][0], acc[mb][1]);
        if (!has_next) break;
        item = next;
        cur = nxt;
    }
}

// ------------------------------------------------------------------ bf16, wide dense form
// Dense fp32-output GEMM over many tiles (the YvMoEGate projection at prefill): out[N][ldo] =
// x[N][K] · Wᵀ (+ a column bias), W [ncols][K] bf16 in the 16 x 64 block order.
//
// One work-group of four wavefronts per 256 x 256 output tile, a 2 x 2 grid of wavefronts
// that each own 128 rows x 128 columns: 8 x 8 blocks of v_mfma_f32_16x16x32_bf16, 256 fp32
// accumulators per lane in AGPRs (an MFMA in inline assembly with the accumulator as one tied
// AGPR operand: the builtin form let the register allocator copy the accumulators between
// AGPRs on every K step). A wavefront reads 16 activation and 16 weight fragments per 64-wide
// chunk for 128 MFMAs (256 LDS bytes per MFMA; the 16-wavefront tile reads 640). Chunks move
// HBM -> LDS by direct loads through a 2-stage ring (2 x 64 KB), the same swizzled activation
// rows and as-stored weight blocks as the 16-wavefront tile. The MFMAs of each chunk run in two
// halves (k = 16 g + 0..7, then 16 g + 8..15, g = lane / 16): the next half's fragment reads
// and, in the second half, the direct loads of chunk c + 2 are spread among them; between the
// halves one barrier frees chunk c's stage and publishes chunk c + 1.
//
// Weights are the MFMA's first operand: a lane's accumulator then holds 4 consecutive output
// columns of one row, stored as one 16-byte non-temporal store (the outputs are read once, by
// another kernel). Measured on the YvMoEGate projection (16,721 x 16,896 x 4,096): the
// element-wise stores of the activations-first order took a quarter of each tile's time, with
// every work-group's epilogue at once; this form runs 7-12 % faster than the 16-wavefront tile.
// Each output accumulates in the 16-wavefront tile's order (chunk by chunk, the k = 16 g + 0..7
// MFMA before the 16 g + 8..15 one), so the results are bit-identical to it.
constexpr int WIDE_K = 64;
__device__ __forceinline__ void dma16s(const void* base, unsigned off, unsigned m0) {
    asm volatile("global_load_lds_dwordx4 %0, %1" : : "v"(off), "s"(base), "{m0}"(m0) : "memory");
}
__device__ __forceinline__ void mfma_acc(f32x4& acc, const bf16x8& a, const bf16x8& b) {
    asm volatile("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(acc) : "v"(a), "v"(b));
}
// s_waitcnt immediate that waits for lgkmcnt <= n only (vmcnt and expcnt at their maxima)
constexpr int lgkm_only(int n) { return 0xf | (0x3 << 14) | (0x7 << 4) | ((n & 0xf) << 8); }

__global__ __launch_bounds__(256) void gemm_wide_kernel(GemmParams p, int ncb) {
    constexpr int MBW = 8, NBW = 8;          // 16-row / 16-column blocks per wavefront
    constexpr int T = MBW * NBW, R = MBW + NBW;  // MFMAs and fragment reads per half chunk
    constexpr int A_BYTES = TBM * WIDE_K * 2, B_BYTES = TBN * WIDE_K * 2;
    constexpr int DA = A_BYTES / 1024 / 4, DB = B_BYTES / 1024 / 4;  // 1 KB loads per wavefront
    __shared__ __attribute__((aligned(1024))) unsigned char lds_a[2][A_BYTES];
    __shared__ __attribute__((aligned(1024))) unsigned char lds_b[2][B_BYTES];
    const int lane = threadIdx.x & 63;
    // uniform in the wavefront (readfirstlane): the direct loads take their base from SGPRs
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wr = wave >> 1, wc = wave & 1;  // 128-row half, 128-column half
    // items (row tile, column block), column block fastest, in 8 contiguous ranges (one per XCD)
    const int ntl = (p.nrows + TBM - 1) / TBM;
    const int total = ntl * ncb;
    const int per_xcd = (total + 7) / 8;
    const int local = blockIdx.x / 8;
    if (local >= per_xcd) return;
    const int item = (blockIdx.x % 8) * per_xcd + local;
    if (item >= total) return;
    const int row0 = (item / ncb) * TBM;
    const int n0 = (item % ncb) * TBN;
    const int nks = p.K / WIDE_K;

    // activation block j of this wavefront: tile rows 8 (DA w + j) .. + 7, lane L row + L / 8,
    // logical chunk (L % 8) ^ (L / 8) ^ (block & 1) (the 16-wavefront tile's swizzle); rows
    // past the batch re-read row 0 of the tile (their results are not stored). 32-bit byte
    // offsets from x (the host checks N * lda * 2 < 2^31).
    unsigned a_off[DA];
#pragma unroll
    for (int j = 0; j < DA; ++j) {
        const int blk = wave * DA + j;
        const int r = blk * 8 + lane / 8;
        const int lc = (lane % 8) ^ (lane / 8) ^ (blk & 1);
        const int gr = (row0 + r < p.nrows) ? row0 + r : row0;
        a_off[j] = (unsigned)((gr * p.lda + lc * 8) * 2);
    }
    // weight 1 KB pieces: piece j = half (j & 1) of the 2 KB block of tile columns
    // 16 (DB w + j) / 2 .. + 15, landing at (DB w + j) KB; the block's base is uniform
    const long long b_rowblk = (long long)(p.K / 64) * 2048;  // bytes between 16-column blocks
    const char* b_base = (const char*)p.B0 + ((n0 >> 4) + wave * (DB / 2)) * b_rowblk;
    const unsigned b_off = (unsigned)lane * 16;
    const unsigned a_lds = (unsigned)(size_t)(lds_ptr_t)&lds_a[0][0] + wave * DA * 1024;
    const unsigned b_lds = (unsigned)(size_t)(lds_ptr_t)&lds_b[0][0] + wave * DB * 1024;
    auto dma = [&](int c, int st, int j) {  // direct load j (activation pieces first) of chunk c
        if (j < DA) {
            dma16s((const char*)p.A + (size_t)c * WIDE_K * 2, a_off[j], a_lds + st * A_BYTES + j * 1024);
        } else {
            const int jb = j - DA;
            dma16s(b_base + (size_t)c * 2048 + (jb >> 1) * b_rowblk + (jb & 1) * 1024, b_off,
                   b_lds + st * B_BYTES + jb * 1024);
        }
    };
    // fragment reads (k group g = lane / 16): activation rows wr 128 + 16 mb + lane % 16, weight
    // rows (output columns) 16 (wc NBW + nb) + lane % 16
    const int g = lane >> 4;
    const int a_rd0 = swz_a(wr * 128 + (lane & 15), 2 * g);
    const int a_rd1 = swz_a(wr * 128 + (lane & 15), 2 * g + 1);
    const int b_rd0 = (wc * NBW) * 2048 + (16 * g + (lane & 15)) * 16;

    f32x4 acc[MBW][NBW];
#pragma unroll
    for (int mb = 0; mb < MBW; ++mb)
#pragma unroll
        for (int nb = 0; nb < NBW; ++nb) acc[mb][nb] = f32x4{0.f, 0.f, 0.f, 0.f};
    bf16x8 fa[2][MBW], fb[2][NBW];  // fragments of the two halves
    auto read_frag = [&](int st, int h, int q) {  // weight fragments first, then activations
        if (q < NBW) fb[h][q] = *(const bf16x8*)(&lds_b[st][0] + b_rd0 + q * 2048 + h * 1024);
        else fa[h][q - NBW] = *(const bf16x8*)(&lds_a[st][0] + (h ? a_rd1 : a_rd0) + (q - NBW) * 16 * 128);
    };
#pragma unroll
    for (int j = 0; j < DA + DB; ++j) dma(0, 0, j);
#pragma unroll
    for (int j = 0; j < DA + DB; ++j) dma(min(1, nks - 1), 1, j);
    __builtin_amdgcn_s_waitcnt(vmcnt_only(DA + DB));  // chunk 0's loads
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
#pragma unroll
    for (int q = 0; q < R; ++q) read_frag(0, 0, q);
    for (int c = 0; c < nks; ++c) {
        const int st = c & 1;
        // half 0 of chunk c; half 1's fragments of chunk c go out meanwhile. MFMA i takes
        // weight block i / 8 and activation block i % 8, so 8 in a row share their first operand.
#pragma unroll
        for (int i = 0; i < T; ++i) {
            mfma_acc(acc[i % MBW][i / MBW], fb[0][i / MBW], fa[0][i % MBW]);
#pragma unroll
            for (int q = (i * R) / T; q < ((i + 1) * R) / T; ++q) read_frag(st, 1, q);
        }
        // every wavefront has read chunk c (its LDS reads done) and holds its loads of chunk
        // c + 1: the barrier frees stage st for chunk c + 2 and publishes chunk c + 1
        __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
        __builtin_amdgcn_s_waitcnt(lgkm_only(0));  // the builtin: the compiler's count knows it
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
        // half 1 of chunk c; half 0's fragments of chunk c + 1 and the direct loads of chunk
        // c + 2 go out meanwhile (past the last chunk the reads see the idle stage and are not
        // used, and the loads repeat the last chunk)
        const int cn = min(c + 2, nks - 1);
#pragma unroll
        for (int i = 0; i < T; ++i) {
            mfma_acc(acc[i % MBW][i / MBW], fb[1][i / MBW], fa[1][i % MBW]);
#pragma unroll
            for (int q = (i * R) / T; q < ((i + 1) * R) / T; ++q) read_frag(st ^ 1, 0, q);
#pragma unroll
            for (int j = (i * (DA + DB)) / T; j < ((i + 1) * (DA + DB)) / T; ++j) dma(cn, st, j);
        }
    }
    // the repeated loads of the last iterations land before the work-group ends; wait states
    // between the last MFMAs and the reads of their accumulators
    __builtin_amdgcn_s_waitcnt(vmcnt_only(0));
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
    // epilogue: the accumulator of block (mb, nb) holds row 16 mb + lane % 16 and the 4
    // consecutive columns 16 nb + 4 g .. + 3
#pragma unroll
    for (int nb = 0; nb < NBW; ++nb) {
        const int n = n0 + (wc * NBW + nb) * 16 + 4 * g;
        f32x4 bias = f32x4{0.f, 0.f, 0.f, 0.f};
        if (p.col_bias != nullptr) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                if (n + i < p.col_bias_n) bias[i] = p.col_bias[n + i];
        }
#pragma unroll
        for (int mb = 0; mb < MBW; ++mb) {
            const int r = row0 + wr * 128 + mb * 16 + (lane & 15);
            if (r < p.nrows) {
                f32x4 v = acc[mb][nb];
                if (p.col_bias != nullptr) {
#pragma unroll
                    for (int i = 0; i < 4; ++i)
                        if (n + i < p.col_bias_n) v[i] = v[i] + bias[i];
                }
                __builtin_nontemporal_store(v, (f32x4*)((float*)p.out + (long long)r * p.ldo + n));
            }
        }
    }
}

// ------------------------------------------------------------------ fp32 activations
// fp32 activations and fp32 weights (the reference's fp32 configuration).
template <int EPI, int NCB>
__global__ __launch_bounds__(256) void gemm_f32_kernel(GemmParams p) {
    constexpr int NM = NMat<EPI>::value;
    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    int e = 0, row0, seg_end;
    if (p.tile_seg != nullptr) {
        const int tile = blockIdx.x;
        if (tile >= *p.ntiles) return;
        e = p.tile_seg[tile];
        row0 = p.tile_row0[tile];
        seg_end = p.seg_start[e + 1];
    } else {
        row0 = blockIdx.x * kTileRows;
        if (row0 >= p.nrows) return;
        seg_end = p.nrows;
    }
    const int col0 = (blockIdx.y * 4 + wave) * NCB * 16;
    if (col0 >= p.ncols) return;
    const int nrb = min(4, (seg_end - row0 + 15) / 16);
    const int kl = (lane >> 4) * 4;
    const int kbeg = blockIdx.z * p.kchunk;
    const int kend = min(p.K, kbeg + p.kchunk);
    const float* arow[4];
#pragma unroll
    for (int rb = 0; rb < 4; ++rb) {
        int r = row0 + rb * 16 + (lane & 15);
        if (r >= seg_end) r = row0;
        arow[rb] = (const float*)p.A + (long long)map_row(p, r) * p.lda + kl;
    }
    const long long e_off = (long long)e * p.b_stride;
    const float* bptr[NM][NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
        const int n = col0 + cb * 16 + (lane & 15);
        bptr[0][cb] = (const float*)p.B0 + e_off + (long long)n * p.K + kl;
        if constexpr (NM == 2) bptr[NM - 1][cb] = (const float*)p.B1 + e_off + (long long)n * p.K + kl;
    }
    f32x4 acc[NM][NCB][4];
#pragma unroll
    for (int m = 0; m < NM; ++m)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
            for (int rb = 0; rb < 4; ++rb) acc[m][cb][rb] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int k0 = kbeg; k0 < kend; k0 += 16) {
        float4 bv[NM][NCB];
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb) bv[m][cb] = *(const float4*)(bptr[m][cb] + k0);
        float4 av[4];
#pragma unroll
        for (int rb = 0; rb < 4; ++rb)
            if (rb < nrb) av[rb] = *(const float4*)(arow[rb] + k0);
#pragma unroll
        for (int m = 0; m < NM; ++m)
#pragma unroll
            for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
                for (int rb = 0; rb < 4; ++rb) {
                    if (rb < nrb) {
                        f32x4& d = acc[m][cb][rb];
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(av[rb].x, bv[m][cb].x, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(av[rb].y, bv[m][cb].y, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(av[rb].z, bv[m][cb].z, d, 0, 0, 0);
                        d = __builtin_amdgcn_mfma_f32_16x16x4f32(av[rb].w, bv[m][cb].w, d, 0, 0, 0);
                    }
                }
    }
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
        const int n = col0 + cb * 16 + (lane & 15);
#pragma unroll
        for (int rb = 0; rb < 4; ++rb) {
            if (rb < nrb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int r = row0 + rb * 16 + (lane >> 4) * 4 + i;
                    if (r < seg_end) {
                        float v;
                        if constexpr (EPI == EPI_SWIGLU) v = silu(acc[0][cb][rb][i]) * acc[NM - 1][cb][rb][i];
                        else if constexpr (EPI == EPI_F32) v = f32_out(p, acc[0][cb][rb][i], n, blockIdx.z);
                        else v = acc[0][cb][rb][i];
                        ((float*)p.out)[blockIdx.z * p.split_stride + (long long)r * p.ldo + n] = v;
                    }
                }
            }
        }
    }
}

// --------------------------------------------------------------- tile schedule
// Segments: routed experts [0, E) from the routing offsets, then S shared experts of N
// rows each after the N*k routed rows. Every segment is cut into tile_rows-row tiles (seg_tiles);
// with light > 0 a remainder of at most light rows goes to the light table instead (seg_light).
__global__ __launch_bounds__(512) void build_tiles_kernel(const int* __restrict__ offsets, int E,
                                                          int S, int N, int k, int tile_rows,
                                                          int fold, int* __restrict__ seg,
                                                          int* __restrict__ tile_seg,
                                                          int* __restrict__ tile_row0,
                                                          int* __restrict__ ntiles, int light,
                                                          int* __restrict__ ltile_seg,
                                                          int* __restrict__ ltile_row0,
                                                          int* __restrict__ lntiles) {
    __shared__ int sc[512];
    __shared__ int lc[512];
    const int tid = threadIdx.x;
    const int nseg = E + S;
    int s0 = 0, s1 = 0, nt = 0, nl = 0;
    if (tid < nseg) {
        if (tid < E) {
            s0 = offsets[tid];
            s1 = offsets[tid + 1];
        } else {
            s0 = N * k + (tid - E) * N;
            s1 = s0 + N;
        }
        seg[tid] = s0;
        if (tid == nseg - 1) seg[nseg] = s1;
        nt = seg_tiles(s1 - s0, tile_rows, fold, light);
        nl = seg_light(s1 - s0, tile_rows, fold, light);
    }
    sc[tid] = nt;
    lc[tid] = nl;
    __syncthreads();
    for (int o = 1; o < 512; o <<= 1) {
        const int v = (tid >= o) ? sc[tid - o] : 0;
        const int u = (tid >= o) ? lc[tid - o] : 0;
        __syncthreads();
        sc[tid] += v;
        lc[tid] += u;
        __syncthreads();
    }
    if (tid < nseg) {
        const int start = sc[tid] - nt;
        for (int q = 0; q < nt; ++q) {
            tile_seg[start + q] = tid;
            tile_row0[start + q] = s0 + q * tile_rows;
        }
        if (nl) {  // the remainder after the segment's full tiles
            ltile_seg[lc[tid] - 1] = tid;
            ltile_row0[lc[tid] - 1] = s0 + ((s1 - s0) / tile_rows) * tile_rows;
        }
    }
    if (tid == 511) {
        *ntiles = sc[511];
        if (light > 0) *lntiles = lc[511];
    }
}

// --------------------------------------------------------------- combine
template <int ACT>
__device__ __forceinline__ float rnd(float x) {
    if constexpr (ACT == YVMOE_ACT_BF16) return round_bf16(x);
    else return x;
}

// out[t] = round( (sum_j w[t,j] * y[pos[t,j]] + shared[t]) + 0.1 * skip[t] ), fp32 sums in
// a fixed order (deterministic, unlike the reference's atomic index_add_ on GPU).
template <int ACT>
__global__ __launch_bounds__(256) void combine_kernel(const void* __restrict__ y, int N, int H,
                                                      int k, int S, const float* __restrict__ w,
                                                      const int* __restrict__ pos,
                                                      const float* __restrict__ mix,
                                                      const void* __restrict__ skip,
                                                      void* __restrict__ out,
                                                      void* __restrict__ shared_out) {
    // the sums below are specified operation by operation (slot order j = 0..k-1, separate
    // multiply and add) so the CPU oracle reproduces them exactly
#pragma clang fp contract(off)
    constexpr int VEC = (ACT == YVMOE_ACT_BF16) ? 8 : 4;
    const int t = blockIdx.y;
    const int h = (blockIdx.x * blockDim.x + threadIdx.x) * VEC;
    if (h >= H) return;
    float acc[VEC], sh[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) {
        acc[v] = 0.0f;
        sh[v] = 0.0f;
    }
    // Rows are loaded KC at a time, all in flight together, then summed in slot order: the
    // arithmetic is the same as a load-then-add loop, without one memory round trip per slot.
    constexpr int KC = 8;
    typedef typename std::conditional<ACT == YVMOE_ACT_BF16, uint4, float4>::type Raw;
    // every expert-output row is read by exactly one token: non-temporal loads
    auto raw_load = [&](long long row) -> Raw {
        if constexpr (ACT == YVMOE_ACT_BF16) {
            return nt_load16((const char*)((const unsigned short*)y + row * H + h));
        } else {
            const u32x4 v = __builtin_nontemporal_load((const u32x4*)((const float*)y + row * H + h));
            return make_float4(__uint_as_float(v.x), __uint_as_float(v.y), __uint_as_float(v.z), __uint_as_float(v.w));
        }
    };
    auto unpack = [&](const Raw& q, float* dst) {
        if constexpr (ACT == YVMOE_ACT_BF16) {
            const unsigned u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                dst[2 * i] = __uint_as_float(u[i] << 16);
                dst[2 * i + 1] = __uint_as_float(u[i] & 0xffff0000u);
            }
        } else {
            dst[0] = q.x;
            dst[1] = q.y;
            dst[2] = q.z;
            dst[3] = q.w;
        }
    };
    float tmp[VEC];
    // the loads that do not wait on the routing (the first KC shared rows and the skip row) go
    // out first, so they travel with the routed rows instead of after them
    Raw qs[KC], qk{};
#pragma unroll
    for (int i = 0; i < KC; ++i)
        if (i < S) qs[i] = raw_load((long long)N * k + (long long)i * N + t);
    if (skip != nullptr) {
        if constexpr (ACT == YVMOE_ACT_BF16) qk = *(const uint4*)((const unsigned short*)skip + (long long)t * H + h);
        else qk = *(const float4*)((const float*)skip + (long long)t * H + h);
    }
    // a slot without a position (pos < 0: an expert id outside [0, E) handed to the dispatch
    // entry) has no expert output and adds nothing
    for (int j0 = 0; j0 < k; j0 += KC) {
        float wj[KC];
        Raw q[KC];
        bool live[KC];
#pragma unroll
        for (int i = 0; i < KC; ++i) {
            live[i] = false;
            if (j0 + i < k) {
                const long long sl = (long long)t * k + j0 + i;
                const int pr = pos[sl];
                live[i] = pr >= 0;
                wj[i] = w[sl];
                if (live[i]) q[i] = raw_load(pr);
            }
        }
#pragma unroll
        for (int i = 0; i < KC; ++i) {
            if (live[i]) {
                unpack(q[i], tmp);
#pragma unroll
                for (int v = 0; v < VEC; ++v) acc[v] = acc[v] + wj[i] * tmp[v];
            }
        }
    }
    for (int s0 = 0; s0 < S; s0 += KC) {
        Raw q[KC];
#pragma unroll
        for (int i = 0; i < KC; ++i)
            if (s0 + i < S) q[i] = s0 == 0 ? qs[i] : raw_load((long long)N * k + (long long)(s0 + i) * N + t);
#pragma unroll
        for (int i = 0; i < KC; ++i) {
            if (s0 + i < S) {
                const float ms = mix[s0 + i];
                unpack(q[i], tmp);
#pragma unroll
                for (int v = 0; v < VEC; ++v) sh[v] = rnd<ACT>(sh[v] + rnd<ACT>(ms * tmp[v]));
            }
        }
    }
    // routed output rounded to the layer dtype, shared mixture and residual sums rounded
    // after every step, as the reference's tensors of that dtype are (layer.py:859-863,
    // :942-945, :750-752)
    float o[VEC];
#pragma unroll
    for (int v = 0; v < VEC; ++v) o[v] = rnd<ACT>(rnd<ACT>(acc[v]) + sh[v]);
    if (skip != nullptr) {
        if constexpr (ACT == YVMOE_ACT_BF16) {
            const uint4 q = qk;
            const unsigned u[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                o[2 * i] = rnd<ACT>(o[2 * i] + rnd<ACT>(0.1f * __uint_as_float(u[i] << 16)));
                o[2 * i + 1] = rnd<ACT>(o[2 * i + 1] + rnd<ACT>(0.1f * __uint_as_float(u[i] & 0xffff0000u)));
            }
        } else {
            const float4 q = qk;
            o[0] = o[0] + 0.1f * q.x;
            o[1] = o[1] + 0.1f * q.y;
            o[2] = o[2] + 0.1f * q.z;
            o[3] = o[3] + 0.1f * q.w;
        }
    }
    if constexpr (ACT == YVMOE_ACT_BF16) {
        unsigned pk[4], ps[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            pk[i] = (unsigned)f32_to_bf16_rne(o[2 * i]) | ((unsigned)f32_to_bf16_rne(o[2 * i + 1]) << 16);
            ps[i] = (unsigned)f32_to_bf16_rne(sh[2 * i]) | ((unsigned)f32_to_bf16_rne(sh[2 * i + 1]) << 16);
        }
        *(uint4*)((unsigned short*)out + (long long)t * H + h) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
        if (shared_out != nullptr)
            *(uint4*)((unsigned short*)shared_out + (long long)t * H + h) = make_uint4(ps[0], ps[1], ps[2], ps[3]);
    } else {
        *(float4*)((float*)out + (long long)t * H + h) = make_float4(o[0], o[1], o[2], o[3]);
        if (shared_out != nullptr)
            *(float4*)((float*)shared_out + (long long)t * H + h) = make_float4(sh[0], sh[1], sh[2], sh[3]);
    }
}

// Sums split-K partial results in split order (deterministic): out[i] = sum_z part[z][i].
__global__ __launch_bounds__(256) void reduce_splits_kernel(const float* __restrict__ part, int nsplit,
                                                            long long stride, long long n,
                                                            float* __restrict__ out) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n) return;
    float s = part[i];
    for (int z = 1; z < nsplit; ++z) s = s + part[(long long)z * stride + i];
    out[i] = s;
}
// The same over four consecutive elements per thread (n and stride multiples of 4, 16-byte
// aligned arrays): each element sums its splits in the same order.
__global__ __launch_bounds__(256) void reduce_splits4_kernel(const float4* __restrict__ part, int nsplit,
                                                             long long stride4, long long n4,
                                                             float4* __restrict__ out) {
    const long long i = (long long)blockIdx.x * 256 + threadIdx.x;
    if (i >= n4) return;
    float4 s = part[i];
    for (int z = 1; z < nsplit; ++z) {
        const float4 v = part[(long long)z * stride4 + i];
        s.x = s.x + v.x;
        s.y = s.y + v.y;
        s.z = s.z + v.z;
        s.w = s.w + v.w;
    }
    out[i] = s;
}
// out[i] = sum over z of part[z * n + i], z in order, for i < n.
int reduce_splits_launch(const float* part, int nsplit, long long n, float* out, hipStream_t st,
                         const char* name) {
    if (n <= 0) return YVMOE_OK;
    if (n % 4 == 0 && ((uintptr_t)part | (uintptr_t)out) % 16 == 0) {
        const long long n4 = n / 4;
        reduce_splits4_kernel<<<(unsigned)((n4 + 255) / 256), 256, 0, st>>>(
            (const float4*)part, nsplit, n4, n4, (float4*)out);
    } else {
        reduce_splits_kernel<<<(unsigned)((n + 255) / 256), 256, 0, st>>>(part, nsplit, n, n, out);
    }
    YV_LAUNCH_CHECK(name);
    return YVMOE_OK;
}

// Streaming (decode) form: one (tile, column group) item per work-group; NB 16-column
// blocks per wavefront.
template <int EPI, int U, int NB, int MAXRB = 1, bool PF = false, int WV = 4, bool WS = false>
int stream_dispatch(int wf, const GemmParams& p, int ntiles_max, hipStream_t st, const char* name,
                    int nsplit = 1) {
    const int ngroups = (EPI == EPI_SWIGLU) ? ceil_div(p.ncols, 8 * WV * NB) : ceil_div(p.ncols, 16 * WV * NB);
    long long items = 8LL * ceil_div(ntiles_max * ngroups * nsplit, 8);
    if constexpr (WS) items += (long long)p.nshared * ceil_div(p.ntok, 64) * ngroups * nsplit;
    if (items <= 0) return YVMOE_OK;
#define YV_ST(WFV) gemm_stream_kernel<WFV, EPI, U, MAXRB, NB, PF, WV, WS><<<(unsigned)items, 64 * WV, 0, st>>>(p, ngroups, nsplit)
    if constexpr (EPI == EPI_F32) {  // dense fp32 output: bf16 weights only
        if (wf != YVMOE_W_BF16) {
            set_error("%s: fp32-output streaming form needs bf16 weights", name);
            return YVMOE_ERR_DTYPE;
        }
        YV_ST(YVMOE_W_BF16);
        YV_LAUNCH_CHECK(name);
        return YVMOE_OK;
    }
    switch (wf) {
        case YVMOE_W_BF16: YV_ST(YVMOE_W_BF16); break;
        case YVMOE_W_INT8: YV_ST(YVMOE_W_INT8); break;
        case YVMOE_W_INT4: YV_ST(YVMOE_W_INT4); break;
        case YVMOE_W_FP8: YV_ST(YVMOE_W_FP8); break;
        default: set_error("unsupported weight format %d for bf16 activations", wf); return YVMOE_ERR_DTYPE;
    }
#undef YV_ST
    YV_LAUNCH_CHECK(name);
    return YVMOE_OK;
}

// LDS-tiled (prefill) form: one work-group per (256-row tile, column block of 128 (gate/up)
// or 256 (down)); grid = 8 x per-XCD range, sized for the most tiles the batch can have.
// fold: the tile table folds remainders (tile_fold), so the form with folded rows runs.
template <int EPI, bool FOLD>
int tile_launch(int wf, const GemmParams& p, int ntiles_max, hipStream_t st, const char* name);

template <int EPI>
int tile_dispatch(int wf, const GemmParams& p, int ntiles_max, hipStream_t st, const char* name,
                  bool fold = false) {
    if constexpr (EPI != EPI_F32) {  // the dense fp32-output form has no tile table
        if (fold) return tile_launch<EPI, true>(wf, p, ntiles_max, st, name);
    }
    return tile_launch<EPI, false>(wf, p, ntiles_max, st, name);
}

template <int EPI, bool FOLD>
int tile_launch(int wf, const GemmParams& p, int ntiles_max, hipStream_t st, const char* name) {
    const int cols = (EPI == EPI_SWIGLU) ? TBN / 2 : TBN;
    // the fp32-output form takes any multiple of 16 columns (a partial last column block) and
    // K splits of kchunk (a multiple of 64; the last split may be shorter)
    const int cmul = EPI == EPI_F32 ? 16 : cols;
    if (p.ncols % cmul != 0 || p.K % TBK != 0 || (EPI == EPI_F32 && (p.kchunk <= 0 || p.kchunk % TBK != 0))) {
        set_error("%s: tiled form needs columns %% %d == 0 and K %% %d == 0 (K=%d, kchunk=%d)", name,
                  cmul, TBK, p.K, p.kchunk);
        return YVMOE_ERR_SHAPE;
    }
    if (ntiles_max <= 0) return YVMOE_OK;
    const int ncb = ceil_div(p.ncols, cols);
    const int nsplit = EPI == EPI_F32 ? ceil_div(p.K, p.kchunk) : 1;
    const long long blocks = 8LL * ceil_div(ntiles_max * ncb * nsplit, 8);
    if (EPI == EPI_F32 && (p.tile_seg != nullptr || wf != YVMOE_W_BF16)) {
        set_error("%s: the fp32-output tiled form is dense with bf16 weights", name);
        return YVMOE_ERR_UNSUPPORTED;
    }
    if constexpr (EPI == EPI_F32) {
        // a grid that fills the chip with whole column blocks and no K split (and whose
        // activation offsets fit 31 bits) takes the wide four-wavefront form; fewer tiles (the
        // router GEMM) keep 16 wavefronts per CU
        if (ntiles_max * ncb >= 256 && (long long)p.nrows * p.lda * 2 < (1ll << 31) && nsplit == 1 &&
            p.ncols % TBN == 0)
            gemm_wide_kernel<<<(unsigned)blocks, 256, 0, st>>>(p, ncb);
        else
            gemm_tile_kernel<YVMOE_W_BF16, EPI><<<(unsigned)blocks, TTHREADS, 0, st>>>(p, ncb);
    } else {
        switch (wf) {
            case YVMOE_W_BF16: gemm_tile_kernel<YVMOE_W_BF16, EPI, 8192, FOLD><<<(unsigned)blocks, TTHREADS, 0, st>>>(p, ncb); break;
            case YVMOE_W_INT8:
                // int8 without folding: 8 wavefronts of 256 x 32 (cfg3 FFN 4.61-4.62 -> 4.55-4.56 ms,
                // same bits; fp8 measured 1.7 % slower on that form, cfg5), one persistent
                // work-group per CU (YV_PTILE)
                if constexpr (!FOLD) {
                    if ((YV_PTILE == 2 || (YV_PTILE == 1 && EPI == EPI_DOWN)) && p.K / TBK >= 3)
                        gemm_tile_persist_kernel<YVMOE_W_INT8, EPI><<<(unsigned)std::min<long long>(blocks, 256), 512, 0, st>>>(p, ncb);
                    else
                        gemm_tile_kernel<YVMOE_W_INT8, EPI, 8192, false, 8><<<(unsigned)blocks, 512, 0, st>>>(p, ncb);
                } else
                    gemm_tile_kernel<YVMOE_W_INT8, EPI, 8192, FOLD><<<(unsigned)blocks, TTHREADS, 0, st>>>(p, ncb);
                break;
            case YVMOE_W_FP8:
                if constexpr (!FOLD) {
                    if (YV_PFP8 && p.K / TBK >= 3 && p.K <= 8192) {
                        gemm_tile_persist_kernel<YVMOE_W_FP8, EPI><<<(unsigned)std::min<long long>(blocks, 256), 512, 0, st>>>(p, ncb);
                        break;
                    }
                }
                gemm_tile_kernel<YVMOE_W_FP8, EPI, 8192, FOLD><<<(unsigned)blocks, TTHREADS, 0, st>>>(p, ncb);
                break;
            case YVMOE_W_INT4:
                if (p.K > 8192) {  // the group-scale table in LDS holds K / 128 <= 64 groups
                    set_error("%s: tiled int4 form needs K <= 8192 (K=%d)", name, p.K);
                    return YVMOE_ERR_SHAPE;
                }
                if constexpr (FOLD) {
                    if (p.K <= 5120)  // 40 scale groups beside a 3-stage ring
                        gemm_tile_kernel<YVMOE_W_INT4, EPI, 5120, true><<<(unsigned)blocks, TTHREADS, 0, st>>>(p, ncb);
                    else              // 64 groups beside a 2-stage ring
                        gemm_tile_kernel<YVMOE_W_INT4, EPI, 8192, true><<<(unsigned)blocks, TTHREADS, 0, st>>>(p, ncb);
                } else {
                    gemm_tile_kernel<YVMOE_W_INT4, EPI, 8192, false><<<(unsigned)blocks, TTHREADS, 0, st>>>(p, ncb);
                }
                break;
            default: set_error("%s: no tiled form for weight format %d", name, wf); return YVMOE_ERR_DTYPE;
        }
    }
    YV_LAUNCH_CHECK(name);
    return YVMOE_OK;
}

// Launches one GEMM: grid (tiles, column groups, K splits); NCB 16-column blocks per wave.
template <int EPI>
int gemm_dispatch(int act, int wf, GemmParams p, int ntiles_max, int ncb, int ksplit,
                  hipStream_t st, const char* name, int maxrb = 4) {
    if (ntiles_max <= 0) return YVMOE_OK;
    if (p.ncols % (16 * ncb) != 0) {
        set_error("%s: %d columns are not a multiple of %d", name, p.ncols, 16 * ncb);
        return YVMOE_ERR_SHAPE;
    }
    const int cols_per_wg = 4 * ncb * 16;
    dim3 grid(ntiles_max, (p.ncols + cols_per_wg - 1) / cols_per_wg, ksplit);
    if (act == YVMOE_ACT_F32) {
        if (ncb == 2) gemm_f32_kernel<EPI, 2><<<grid, 256, 0, st>>>(p);
        else gemm_f32_kernel<EPI, 1><<<grid, 256, 0, st>>>(p);
    } else {
#define YV_GB(WFV)                                                                  \
    do {                                                                            \
        if (maxrb == 1) {                                                           \
            if (ncb == 2) gemm_bf16_kernel<WFV, EPI, 2, 1><<<grid, 256, 0, st>>>(p); \
            else gemm_bf16_kernel<WFV, EPI, 1, 1><<<grid, 256, 0, st>>>(p);         \
        } else {                                                                    \
            if (ncb == 2) gemm_bf16_kernel<WFV, EPI, 2, 4><<<grid, 256, 0, st>>>(p); \
            else gemm_bf16_kernel<WFV, EPI, 1, 4><<<grid, 256, 0, st>>>(p);         \
        }                                                                           \
    } while (0)
        switch (wf) {
            case YVMOE_W_BF16: YV_GB(YVMOE_W_BF16); break;
            case YVMOE_W_INT8: YV_GB(YVMOE_W_INT8); break;
            case YVMOE_W_INT4: YV_GB(YVMOE_W_INT4); break;
            case YVMOE_W_FP8: YV_GB(YVMOE_W_FP8); break;
            default: set_error("unsupported weight format %d for bf16 activations", wf); return YVMOE_ERR_DTYPE;
        }
#undef YV_GB
    }
    YV_LAUNCH_CHECK(name);
    return YVMOE_OK;
}

}  // namespace

int dense_gemm_launch(const void* x, int act, int N, int K, const void* w, int ncols, float* out,
                      int ld, float* partials, hipStream_t st, const char* name) {
    if (N <= 0) return YVMOE_OK;
    GemmParams p{};
    p.A = x;
    p.lda = K;
    p.rowmap = nullptr;
    p.B0 = w;
    p.K = K;
    p.ncols = ncols;
    p.ldo = ld;
    p.nrows = N;
    const int wf = (act == YVMOE_ACT_F32) ? YVMOE_W_F32 : YVMOE_W_BF16;
    if (dense_tiled(act, N, ncols, K)) {
        p.kchunk = K;
        p.out = out;
        return tile_dispatch<EPI_F32>(wf, p, ceil_div(N, TBM), st, name);
    }
    const int ks = dense_ksplit(N, ncols, K);
    const int ncb = (ncols % 32 == 0) ? 2 : 1;
    if (ks == 1 || partials == nullptr) {
        p.kchunk = K;
        p.out = out;
        return gemm_dispatch<EPI_F32>(act, wf, p, ceil_div(N, kTileRows), ncb, 1, st, name);
    }
    p.kchunk = K / ks;
    p.out = partials;
    p.split_stride = (long long)N * ld;
    int rc = gemm_dispatch<EPI_F32>(act, wf, p, ceil_div(N, kTileRows), ncb, ks, st, name);
    if (rc) return rc;
    return reduce_splits_launch(partials, ks, (long long)N * ld, out, st, "dense_gemm_reduce");
}

int dense_partials_launch(const void* x, int act, int N, int K, const void* w, int ncols,
                          float* out, int ld, const float* col_bias, int col_bias_n,
                          hipStream_t st, const char* name) {
    if (N <= 0) return YVMOE_OK;
    GemmParams p{};
    p.col_bias = col_bias;
    p.col_bias_n = col_bias_n;
    p.A = x;
    p.lda = K;
    p.rowmap = nullptr;
    p.B0 = w;
    p.K = K;
    p.ncols = ncols;
    p.ldo = ld;
    p.nrows = N;
    p.out = out;
    p.split_stride = (long long)N * ld;
    const int ks = dense_splits(act, N, ncols, K);
    p.kchunk = K / ks;
    if (dense_tiled(act, N, ncols, K)) return tile_dispatch<EPI_F32>(YVMOE_W_BF16, p, ceil_div(N, TBM), st, name);
    if (dense_streamed(act, N, ncols, K)) {
        if (N <= 16) return stream_dispatch<EPI_F32, 4, 1, 1>(YVMOE_W_BF16, p, 1, st, name, ks);
        // one k-step per staged chunk with the next chunk's weights in flight: the YvMoEGate
        // decode projection (64 x 4096 x 16,896) 35.1-35.7 -> 33.0-33.6 us against two k-steps
        // (4/8/16 wavefronts, 1-4 column blocks per wavefront and 1-16 K splits measured slower
        // or needing more partial sums)
        return stream_dispatch<EPI_F32, 1, 1, 4, YV_DPF>(YVMOE_W_BF16, p, 1, st, name, ks);
    }
    const int wf = (act == YVMOE_ACT_F32) ? YVMOE_W_F32 : YVMOE_W_BF16;
    return gemm_dispatch<EPI_F32>(act, wf, p, ceil_div(N, kTileRows), (ncols % 32 == 0) ? 2 : 1, ks,
                                  st, name);
}

int router_gemm_launch(const void* x, int act, int N, const yvmoe_router* r, float* out, int ld,
                       float* partials, hipStream_t st, bool reduce) {
    GemmParams p{};
    p.A = x;
    p.lda = r->hidden;
    p.rowmap = nullptr;
    p.B0 = r->w_router;
    p.K = r->hidden;
    p.ncols = router_ld(r->num_experts, act);
    p.ldo = ld;
    p.nrows = N;
    const int wf = (act == YVMOE_ACT_F32) ? YVMOE_W_F32 : YVMOE_W_BF16;
    const int ks = router_ksplit(N, r->num_experts, act, r->hidden);
    if (router_tiled(act, N, p.ncols, r->hidden)) {
        // large batches: the LDS-tiled MFMA form over (tile, column block, K split) items, the
        // split partial sums reduced in split order
        if (ks == 1 || partials == nullptr) {
            p.kchunk = r->hidden;
            p.out = out;
            return tile_dispatch<EPI_F32>(YVMOE_W_BF16, p, ceil_div(N, TBM), st, "router_gemm");
        }
        p.kchunk = router_tiled_steps(N, p.ncols, r->hidden) * 64;
        p.out = partials;
        p.split_stride = (long long)N * ld;
        int rc = tile_dispatch<EPI_F32>(YVMOE_W_BF16, p, ceil_div(N, TBM), st, "router_gemm");
        if (rc || !reduce) return rc;
        return reduce_splits_launch(partials, ks, (long long)N * ld, out, st, "router_reduce");
    }
    p.kchunk = r->hidden / ks;
    if (ks == 1 || partials == nullptr) {
        p.kchunk = r->hidden;
        p.out = out;
        const int ncb = (p.ncols % 32 == 0) ? 2 : 1;
        return gemm_dispatch<EPI_F32>(act, wf, p, ceil_div(N, kTileRows), ncb, 1, st, "router_gemm");
    }
    p.out = partials;
    p.split_stride = (long long)N * ld;
    int rc;
    // up to 64 rows: the weight-streaming form, in 16-row tiles (the router operand, 2 MB at
    // E = 64, stays in L2 for the tiles that re-read it: 2.7 us less per decode step than one
    // 64-row tile; the 138 MB YvMoEGate projection keeps 64-row tiles, which measured faster)
    if (dense_streamed(act, N, p.ncols, r->hidden))
        rc = stream_dispatch<EPI_F32, 4, 1, 1>(YVMOE_W_BF16, p, ceil_div(N, 16), st, "router_gemm", ks);
    else
        rc = gemm_dispatch<EPI_F32>(act, wf, p, ceil_div(N, kTileRows), 1, ks, st, "router_gemm");
    if (rc || !reduce) return rc;
    return reduce_splits_launch(partials, ks, (long long)N * ld, out, st, "router_reduce");
}

int ffn_tile_rows(int act, int N, int k, int E, int H, int F, int wf) {
    // 256-row LDS-tiled form when experts hold many rows (prefill-like batches)
    const bool tiled = act == YVMOE_ACT_BF16 && N * k >= 64 * E && F % (TBN / 2) == 0 && H % TBN == 0 &&
                       (wf == YVMOE_W_INT8 || wf == YVMOE_W_BF16 ||
                        ((wf == YVMOE_W_FP8 || wf == YVMOE_W_INT4) && H <= 8192 && F <= 8192));
    if (tiled) return TBM;
    // 16-row tiles (one MFMA row block per wave) when experts hold few rows (decode-like
    // batches), 64-row tiles otherwise
    return (act == YVMOE_ACT_BF16 && N * k <= 32 * E) ? 16 : 64;
}

TileTable ffn_tile_table(int N, int k, int E, int S, int F, int act, int tile_rows, char* ws) {
    const RouteWs RL = route_ws(N, E, k);
    const FfnWs FL = ffn_ws(N, k, E, S, F, act);
    char* fws = ws + RL.bytes;
    TileTable t;
    t.seg = (int*)(fws + FL.seg);
    t.tile_seg = (int*)(fws + FL.tile_seg);
    t.tile_row0 = (int*)(fws + FL.tile_row0);
    t.ntiles = (int*)(fws + FL.ntiles);
    t.S = S;
    t.tile_rows = tile_rows;
    t.fold = tile_rows == TBM ? tile_fold(N, k, E) : 0;
    t.light = tile_rows == TBM ? tile_light(N, k, E, t.fold) : 0;
    t.ltile_seg = (int*)(fws + FL.lseg);
    t.ltile_row0 = (int*)(fws + FL.lrow0);
    t.lntiles = (int*)(fws + FL.lntiles);
    return t;
}

int expert_ffn_launch(const void* x, int act, int N, int k, const yvmoe_expert_weights* w,
                      const yvmoe_routing* routing, void* y, char* ws, hipStream_t st, bool tiles_ready) {
    const int E = w->num_routed, S = w->num_shared, H = w->hidden, F = w->ffn;
    const RouteWs RL = route_ws(N, E, k);
    const FfnWs FL = ffn_ws(N, k, E, S, F, act);
    char* fws = ws + RL.bytes;
    void* hbuf = fws + FL.h;
    const int tile_rows = ffn_tile_rows(act, N, k, E, H, F, w->format);
    const bool tiled = tile_rows == TBM;
    const int maxrb = tile_rows == 16 ? 1 : 4;
    const TileTable tt = ffn_tile_table(N, k, E, S, F, act, tile_rows, ws);
    int* seg = tt.seg;
    int* tile_seg = tt.tile_seg;
    int* tile_row0 = tt.tile_row0;
    int* ntiles = tt.ntiles;
    const int T = max_tiles(N, k, E, S, tile_rows);
    if (!tiles_ready) {
        build_tiles_kernel<<<1, 512, 0, st>>>(routing->offsets, E, S, N, k, tile_rows, tt.fold, seg,
                                              tile_seg, tile_row0, ntiles, tt.light, tt.ltile_seg,
                                              tt.ltile_row0, tt.lntiles);
        YV_LAUNCH_CHECK("build_tiles");
    } else if (tt.light > 0) {
        set_error("internal: a light tile table is built by the FFN launch itself");
        return YVMOE_ERR_ARG;
    }
    const int wf = w->format;
    // the light table's remainders (at most tt.light rows, one per segment) on the streaming
    // form with tt.light-row tiles, after the main table's launch of the same GEMM; 32-row
    // tiles with four 16-column blocks per wavefront (a quarter of the activation staging per
    // weight byte: cfg5 FFN -1.9 % against one block), 64-row tiles with one (1, 2 and 4
    // blocks measured alike at cfg4)
    auto light_launch = [&](GemmParams q, auto epi, const char* name) {
        constexpr int EPIV = decltype(epi)::value;
        q.tile_seg = tt.ltile_seg;
        q.tile_row0 = tt.ltile_row0;
        q.ntiles = tt.lntiles;
        if (tt.light > 32) return stream_dispatch<EPIV, 2, 1, 4, true, 4>(wf, q, E + S, st, name);
        return stream_dispatch<EPIV, 2, 4, 2, true, 4>(wf, q, E + S, st, name);
    };
    GemmParams p{};
    p.tile_seg = tile_seg;
    p.tile_row0 = tile_row0;
    p.ntiles = ntiles;
    p.seg_start = seg;
    // GEMM1: h = silu(x Wg^T) * (x Wu^T) over gathered rows
    p.A = x;
    p.lda = H;
    p.rowmap = routing->perm;
    p.rowdiv = k;
    p.routed_rows = N * k;
    p.ntok = N;
    p.nshared = S;
    p.B0 = w->w_gate;
    p.B1 = w->w_up;
    p.S0 = w->s_gate;
    p.S1 = w->s_up;
    p.b_stride = (long long)F * H;
    if (wf == YVMOE_W_INT8) p.s_stride = F;
    else if (wf == YVMOE_W_INT4) p.s_stride = (long long)F * (H / 128);
    else if (wf == YVMOE_W_FP8) p.s_stride = (long long)(F / 128) * (H / 128);
    p.K = H;
    p.ncols = F;
    p.out = hbuf;
    p.ldo = F;
    p.kchunk = H;
    const bool streaming = (maxrb == 1);
    int rc = tiled ? tile_dispatch<EPI_SWIGLU>(wf, p, T, st, "expert_gemm1", tt.fold > 0)
           : streaming ? (S > 0
                              ? stream_dispatch<EPI_SWIGLU, YV_U1, YV_NB1, 1, YV_PF1, YV_WV1, true>(wf, p, T, st, "expert_gemm1")
                              : stream_dispatch<EPI_SWIGLU, YV_U1, YV_NB1, 1, YV_PF1, YV_WV1>(wf, p, T, st, "expert_gemm1"))
                       : gemm_dispatch<EPI_SWIGLU>(act, wf, p, T, (F % 32 == 0) ? 2 : 1, 1, st,
                                                   "expert_gemm1", maxrb);
    if (rc != YVMOE_OK) return rc;
    if (tt.light > 0) {
        rc = light_launch(p, std::integral_constant<int, EPI_SWIGLU>{}, "expert_gemm1_light");
        if (rc != YVMOE_OK) return rc;
    }
    // GEMM2: y = h Wd^T (rows already in sorted order)
    p.A = hbuf;
    p.lda = F;
    p.rowmap = nullptr;
    p.B0 = w->w_down;
    p.B1 = nullptr;
    p.S0 = w->s_down;
    p.S1 = nullptr;
    p.b_stride = (long long)H * F;
    if (wf == YVMOE_W_INT8) p.s_stride = H;
    else if (wf == YVMOE_W_INT4) p.s_stride = (long long)H * (F / 128);
    else if (wf == YVMOE_W_FP8) p.s_stride = (long long)(H / 128) * (F / 128);
    p.K = F;
    p.ncols = H;
    p.out = y;
    p.ldo = H;
    p.kchunk = F;
    if (tiled) {
        rc = tile_dispatch<EPI_DOWN>(wf, p, T, st, "expert_gemm2", tt.fold > 0);
        if (rc != YVMOE_OK || tt.light == 0) return rc;
        return light_launch(p, std::integral_constant<int, EPI_DOWN>{}, "expert_gemm2_light");
    }
    return streaming ? (S > 0
                            ? stream_dispatch<EPI_DOWN, YV_U2, YV_NB2, 1, YV_PF2, YV_WV2, true>(wf, p, T, st, "expert_gemm2")
                            : stream_dispatch<EPI_DOWN, YV_U2, YV_NB2, 1, YV_PF2, YV_WV2>(wf, p, T, st, "expert_gemm2"))
                     : gemm_dispatch<EPI_DOWN>(act, wf, p, T, (H % 32 == 0) ? 2 : 1, 1, st,
                                               "expert_gemm2", maxrb);
}

int combine_launch(const void* y, int act, int N, int H, int k, int S, const yvmoe_routing* routing,
                   const float* mix, const void* skip, void* out, void* shared_out, hipStream_t st) {
    if (N == 0) return YVMOE_OK;
    const int vec = (act == YVMOE_ACT_BF16) ? 8 : 4;
    dim3 grid(ceil_div(H / vec, 256), N);
    if (act == YVMOE_ACT_BF16)
        combine_kernel<YVMOE_ACT_BF16><<<grid, 256, 0, st>>>(y, N, H, k, S, routing->weights,
                                                             routing->pos, mix, skip, out,
                                                             S > 0 ? shared_out : nullptr);
    else
        combine_kernel<YVMOE_ACT_F32><<<grid, 256, 0, st>>>(y, N, H, k, S, routing->weights,
                                                            routing->pos, mix, skip, out,
                                                            S > 0 ? shared_out : nullptr);
    YV_LAUNCH_CHECK("combine");
    return YVMOE_OK;
}

}  // namespace yvmoe
