// W4A4 GEMM of the SVDQuant linears on gfx950 matrix cores.
//
//   y[m][n] = sum_g as[g][m] * ws[g][n] * I_g[m][n]  +  bf16(lora[m]) . pu[n]  +  bias[n]
//   I_g[m][n] = sum_{k in group g} qa[m][k] * qw[n][k]          (exact integers)
//
// Operands: qa — activation int4 values as fp6 codes (wdl_act_quant_w4); wc — weight int4 values as fp6 codes
// (wdl_w4a4_weight_codes, expanded once from the packed [N, K/2] nibbles), both tile-blocked 48 bytes per row
// and 64-deep group (the format is described with blocked6_offset); as [K/64, Mp] bf16; ws [K/64, N] as bf16 pairs
// (hi, lo) with hi + lo = the weight scale exactly (a bf16 scale is (s, 0), an fp16 scale splits into two bf16
// parts: wdl_w4a4_scale_pairs); lora fp32 [Mp, 32]; pu bf16 [N, 32]; bias bf16 [N].
//
// Arithmetic: weights are e3m2 codes of 2w and activations e2m3 codes of q / 2, so v_mfma_f32_32x32x64_f8f6f4 in
// its fp6 x fp6 form (one 64-deep group per instruction, 32 cycles: twice the int8 rate) returns I_g exactly as
// an fp32 integer (|I_g| <= 64 * 8 * 15 < 2^24). The per-group scale product ws[n] * as[m] comes from a bf16
// MFMA with two k-slots, hi as + lo as (exact: each product 8 by 8 significant bits, the sum at most 11 by 8), and
// each group is folded in with one fmaf per element,
// groups in increasing order. The low-rank term is two bf16 MFMAs accumulated into the result, then the bias.
//
// Orientation: the tile is computed transposed, C^T[n][m] (rows = output features, columns = tokens), so a lane
// holds one token and 16 features: row n = 8*(i/4) + 4*(lane/32) + i%4, column m = lane%32 of each 32x32 subtile.
// Both operands arrive as codes, so the main loop issues no conversion work: per MFMA pair its vector ALU work is
// the 16 fmaf of the scale fold.
//
// The FP8 linears (wdl_fp8_gemm) share the main loop with e4m3 codes in plain row-major [rows, K] operands and
// one fp32 accumulation over all of K.
#include "wdl_common.h"

namespace {

using namespace wdl;

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef unsigned u32x6 __attribute__((ext_vector_type(6)));

enum Epilogue {
    EPI_BF16 = 0, EPI_F32 = 1, EPI_RESIDUAL = 2, EPI_GELU = 3, EPI_FP8_ROWS = 4, EPI_FP8_TENSOR = 5,
    EPI_GELU_QUANT = 6  // the fused GELU MLP's first layer: codes, scales and low-rank partials of the second's input
};
constexpr float GELU_SHIFT = 0.171875f;  // quantization/w4a4.py:195: GELU(x) > -0.17, so GELU(x) + shift >= 0

// GELU, tanh form: 0.5 x (1 + tanh(u)), u = sqrt(2/pi) (x + 0.044715 x^3), computed as the identical
// x / (1 + exp(-2u)) with exp(-2u) = 2^(x (C1 + C2 x^2)) on the hardware exp2 and reciprocal (about 1 ulp each).
// Unlike 1 + tanh(u) it does not cancel for negative x. Large negative x: exp -> inf, x * 0 = -0; large positive
// x: exp -> 0, x.
__device__ __forceinline__ float gelu_tanh(float x) {
    constexpr float C1 = -2.0f * 0.7978845608028654f * 1.4426950408889634f;  // -2 sqrt(2/pi) log2(e)
    constexpr float C2 = C1 * 0.044715f;
    const float e = __builtin_amdgcn_exp2f(x * fmaf(C2, x * x, C1));
    return x * __builtin_amdgcn_rcpf(1.0f + e);
}

struct GemmArgs {
    const uint8_t* qa;        // W4A4: fp6 e2m3 codes, tile-blocked [Mp/128][K/64][128][48]; FP8: e4m3 [Mp, K]
    const uint16_t* as;       // [G, Mp]
    const uint8_t* wc;        // W4A4: fp6 e3m2 codes, tile-blocked [N/128][K/64][128][48]; FP8: e4m3 [N, K]
    const uint32_t* ws;       // W4A4: [G, N] weight scale pairs (hi | lo << 16), bf16 parts
    const float* lora;        // [Mp, 32] or null
    const uint16_t* pu;       // [N, 32] or null
    const uint16_t* bias;     // [N] or null
    int64_t M, Mp, N, K;
    void* out;                // bf16 / fp32 [M, ldo]
    int64_t ldo;
    const float* gate;        // [N] fp32 (EPI_RESIDUAL: out += gate * bf16(y))
    const float* xs;          // FP8 linears: activation scales fp32 [Mp] (rows) or [1] (tensor)
    const float* wsf;         // FP8 linears: weight scales fp32 [N] (rows) or [1] (tensor)
    float* part;              // stream-K partial sums (workspace), or null
    // EPI_GELU_QUANT: the second layer's input (the hidden layer, N = its width)
    uint8_t* q2;              // fp6 e2m3 codes of the unsigned int4 values, tile-blocked [Mp/128][N/64][128][48]
    uint16_t* as2;            // bf16 [N/64, Mp]
    const uint16_t* sm2;      // smooth2, bf16 [N]
    const uint16_t* pd2t;     // proj_down2^T, bf16 [32, N]
    float* lpart;             // low-rank partials fp32 [N/128][Mp][32]
    float2* lnp;              // EPI_RESIDUAL: LayerNorm chunk partials of the output rows [M][N / 32], or null
};

// LayerNorm chunk partials of the rows a residual epilogue writes (the activation quantizer's LN input): for a row's
// 32-value chunk, (S, M2) = its sum and its sum of squared deviations from its mean S / 32, each as 8 quads of 4
// values summed in order and the quads combined as ((t0 + t1) + (t2 + t3)) + ((t4 + t5) + (t6 + t7)), on the bf16
// values written. The staged epilogue holds 8 consecutive values per lane (quads 2a, 2a + 1 of a chunk, a = lane
// % 4 of a 4-lane group), the MFMA layout 4 per lane half (quad 2q + half of quarter q).
__device__ __forceinline__ float quad_sum(float a, float b, float c, float d) { return ((a + b) + c) + d; }
__device__ __forceinline__ float quad_sq(float a, float b, float c, float d, float m) {
    const float da = a - m, db = b - m, dc = c - m, dd = d - m;
    return ((da * da + db * db) + dc * dc) + dd * dd;
}

// Tile BN (features) x BM (tokens), NW waves in a (BN / WN) x (BM / WM) grid. Every operand byte streams from
// global memory straight into a STAGES-deep LDS ring with global_load_lds (lane-linear in LDS: 16 or 4 bytes per
// lane), issued STAGES - 1 groups ahead, so no staging registers are involved. Every wave issues the same number
// of these loads per group, so each wave's vmcnt names exactly the groups still in flight; the loads are written
// as inline asm so that the compiler's own wait insertion, which cannot tell the ring stages apart, does not add
// vmcnt(0) waits in front of every LDS read.
//   W4A4: a stage is the group's fp6 weight codes [BN][48 B] then activation codes [BM][48 B] — contiguous 6 KB
//   blocks in global memory — split evenly over the waves, plus the scales: ws[BN] pairs, as[BM]. Rows of 48 bytes
//   read as 16 + 8 bytes per lane are free of bank conflicts on the 16-byte reads. Each scale stage ends in 128 zero
//   bytes that lanes 32..63 read, which zeroes their half of the scale-product operands without a select.
//   FP8: separate activation [BM][64 B] and weight [BN][64 B] stages, code rows with their four 16-byte quarters
//   XOR-swizzled by (row / 4) % 4 (conflict-free operand reads).
// Workgroup ids are remapped so that the tiles of one weight slab run on one XCD.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// 64 lanes x 16 bytes from per-lane global addresses to LDS [m0, m0 + 1024)
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}
// The same from a wave-uniform base (scalar registers) plus a 32-bit per-lane offset: the address arithmetic of a
// load stays on the scalar unit
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}
__device__ __forceinline__ void dma4s(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("global_load_lds_dword %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

// s_waitcnt vmcnt(n) only (expcnt and lgkmcnt left at their maxima)
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Low-rank branch, bias and epilogue of one wave's TN x TM subtiles (rows nb0 + 32 i + .., tokens mb0 + 32 j + ..).
// Every load the epilogue needs (low-rank operands, bias, gate, the residual it updates, FP8 scales) is issued
// before the first store: the output may alias nothing the compiler can see, so loads written between the stores
// would each wait for the previous stores and pay a full memory round trip.
template <int TN, int TM, int EPI>
__device__ __forceinline__ void finish_tile(const GemmArgs& p, f32x16 (&acc)[TN][TM], int64_t nb0, int64_t mb0,
                                            int lane) {
    const int half = lane / 32;
    // ---- loads
    bf16x8 pa[TN][2];
    float4 lr[TM][2][2];
    if (p.lora) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                pa[i][h] = *reinterpret_cast<const bf16x8*>(p.pu + (nb0 + i * 32 + lane % 32) * 32 + h * 16 + 8 * half);
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float* l = p.lora + (mb0 + j * 32 + lane % 32) * 32 + h * 16 + 8 * half;
                lr[j][h][0] = *reinterpret_cast<const float4*>(l);
                lr[j][h][1] = *reinterpret_cast<const float4*>(l + 4);
            }
    }
    // per (i, q): this lane's 4 output features nb = nb0 + 32 i + 8 q + 4 half .. + 3
    uint2 bias[TN][4];
    float4 gate[TN][4];
    float4 wsf[TN][4];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int64_t nb = nb0 + i * 32 + 8 * q + 4 * half;
            bias[i][q] = p.bias ? *reinterpret_cast<const uint2*>(p.bias + nb)
                                : make_uint2(0x80008000u, 0x80008000u);  // -0: an exact identity of the sum
            if (EPI == EPI_RESIDUAL) gate[i][q] = *reinterpret_cast<const float4*>(p.gate + nb);
            if (EPI == EPI_FP8_ROWS) wsf[i][q] = *reinterpret_cast<const float4*>(p.wsf + nb);
        }
    uint2 old[TN][TM][4];
    float xsm[TM];
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int64_t m = mb0 + j * 32 + lane % 32;
        const int64_t mm = m < p.M ? m : 0;  // rows past M read row 0 and are not stored
        if (EPI == EPI_FP8_ROWS) xsm[j] = p.xs[m];
        if (EPI == EPI_RESIDUAL)
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int q = 0; q < 4; ++q)
                    old[i][j][q] = *reinterpret_cast<const uint2*>(static_cast<const uint16_t*>(p.out) + mm * p.ldo +
                                                                   nb0 + i * 32 + 8 * q + 4 * half);
    }
    const float xs0 = EPI == EPI_FP8_TENSOR ? p.xs[0] * p.wsf[0] : 0.0f;
    static_assert(EPI != EPI_RESIDUAL || (TN == 1 && TM == 1), "the gated residual runs here on 32 x 32 pieces only");
    float nx[EPI == EPI_RESIDUAL ? 16 : 1] = {};  // the piece's new values of the lane (LayerNorm partials)

    // ---- low-rank branch: acc += pu[n] . bf16(lora[m]) over r = 0..31, two 32x32x16 bf16 MFMAs per subtile
    if (p.lora) {
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                bf16x8 lb;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    lb[e] = __builtin_bit_cast(__bf16, f32_to_bf16(lr[j][h][0][e]));
                    lb[4 + e] = __builtin_bit_cast(__bf16, f32_to_bf16(lr[j][h][1][e]));
                }
#pragma unroll
                for (int i = 0; i < TN; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[i][h], lb, acc[i][j], 0, 0, 0);
            }
    }

    // ---- epilogue and stores
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const int64_t m = mb0 + j * 32 + lane % 32;
            if (m >= p.M) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t nb = nb0 + i * 32 + 8 * q + 4 * half;
                const uint16_t bv[4] = {uint16_t(bias[i][q].x), uint16_t(bias[i][q].x >> 16), uint16_t(bias[i][q].y),
                                        uint16_t(bias[i][q].y >> 16)};
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y[e] = acc[i][j][4 * q + e];
                    if (EPI == EPI_FP8_ROWS)  // fp8.py:57-62: bf16 product, then * (xs ws) in fp32, + b
                        y[e] = bf16_to_f32(f32_to_bf16(y[e])) * (xsm[j] * wsf[i][q][e]);
                    else if (EPI == EPI_FP8_TENSOR)  // _scaled_mm: acc * (xs ws) + b, one rounding
                        y[e] = y[e] * xs0;
                    y[e] = y[e] + bf16_to_f32(bv[e]);  // -0 without a bias
                }
                if (EPI == EPI_F32) {
                    float* o = static_cast<float*>(p.out) + m * p.ldo + nb;
                    *reinterpret_cast<float4*>(o) = make_float4(y[0], y[1], y[2], y[3]);
                } else {
                    uint16_t* o = static_cast<uint16_t*>(p.out) + m * p.ldo + nb;
                    uint16_t r[4];
                    if (EPI == EPI_RESIDUAL) {
                        const uint2 ow = old[i][j][q];
                        const uint16_t ov[4] = {uint16_t(ow.x), uint16_t(ow.x >> 16), uint16_t(ow.y), uint16_t(ow.y >> 16)};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float yb = bf16_to_f32(f32_to_bf16(y[e]));
                            r[e] = f32_to_bf16(bf16_to_f32(ov[e]) + yb * gate[i][q][e]);
                            if constexpr (EPI == EPI_RESIDUAL) nx[4 * q + e] = bf16_to_f32(r[e]);
                        }
                    } else if (EPI == EPI_GELU) {
#pragma unroll
                        for (int e = 0; e < 4; ++e) r[e] = f32_to_bf16(gelu_tanh(y[e]));
                    } else {
#pragma unroll
                        for (int e = 0; e < 4; ++e) r[e] = f32_to_bf16(y[e]);
                    }
                    *reinterpret_cast<uint2*>(o) = make_uint2(r[0] | (uint32_t(r[1]) << 16), r[2] | (uint32_t(r[3]) << 16));
                }
            }
        }
    if constexpr (EPI == EPI_RESIDUAL) {
        if (p.lnp) {  // the piece's 32 features are one chunk; quarter q of a lane half holds quad 2 q + half
            float t[4], u[4];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                t[q] = quad_sum(nx[4 * q], nx[4 * q + 1], nx[4 * q + 2], nx[4 * q + 3]);
                t[q] = xor_sum<32>(t[q]);  // quads 2 q + 2 q + 1
            }
            const float S = (t[0] + t[1]) + (t[2] + t[3]), mc = S * (1.0f / 32);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                u[q] = quad_sq(nx[4 * q], nx[4 * q + 1], nx[4 * q + 2], nx[4 * q + 3], mc);
                u[q] = xor_sum<32>(u[q]);
            }
            const float M2 = (u[0] + u[1]) + (u[2] + u[3]);
            const int64_t m = mb0 + lane % 32;
            if (half == 0 && m < p.M) p.lnp[m * (p.N / 32) + nb0 / 32] = make_float2(S, M2);
        }
    }
}

// Staged epilogue of the W4A4 GEMM's bf16 outputs (bf16, GELU, gated residual) for a wave's 64 x 64 subtiles.
// The low-rank term, bias and GELU are applied in the MFMA layout (lane = token), the bf16 results go through the
// wave's LDS area, and the output is then read and written token-major: lane l owns features 8 (l % 8) .. + 7 of
// tokens 8 k + l / 8 (k = 0..7), so 8 lanes cover one token's 128 contiguous bytes and every global access is 16
// bytes per lane (in the MFMA layout a store touches 32 rows in 8-byte pieces). The residual rows and the gate
// are loaded first, with the low-rank operands, so their latency overlaps the low-rank MFMAs and the staging.
// Arithmetic as in finish_tile.
constexpr int STG = 64 + 4;  // staged row: 64 bf16 + 4 pad (136 bytes: conflict-free 8-byte writes of 32 rows)
template <int TN, int TM, int EPI>
__device__ __forceinline__ void finish_tile_rows(const GemmArgs& p, f32x16 (&acc)[TN][TM], int64_t nb0, int64_t mb0,
                                                 int lane, uint16_t* stage) {
    static_assert(TN == 2 && TM == 2, "64 x 64 per wave");
    static_assert(EPI == EPI_BF16 || EPI == EPI_RESIDUAL || EPI == EPI_GELU, "bf16 outputs");
    const int half = lane / 32;
    const int rc = lane % 8;  // token-major phase: feature chunk
    // ---- loads
    bf16x8 pa[TN][2];
    float4 lr[TM][2][2];
    if (p.lora) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                pa[i][h] = *reinterpret_cast<const bf16x8*>(p.pu + (nb0 + i * 32 + lane % 32) * 32 + h * 16 + 8 * half);
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float* l = p.lora + (mb0 + j * 32 + lane % 32) * 32 + h * 16 + 8 * half;
                lr[j][h][0] = *reinterpret_cast<const float4*>(l);
                lr[j][h][1] = *reinterpret_cast<const float4*>(l + 4);
            }
    }
    uint2 bias[TN][4];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q)
            bias[i][q] = p.bias ? *reinterpret_cast<const uint2*>(p.bias + nb0 + i * 32 + 8 * q + 4 * half)
                                : make_uint2(0x80008000u, 0x80008000u);  // -0: an exact identity of the sum
    float4 gate[2];
    uint4 old[8];
    if (EPI == EPI_RESIDUAL) {
        gate[0] = *reinterpret_cast<const float4*>(p.gate + nb0 + 8 * rc);
        gate[1] = *reinterpret_cast<const float4*>(p.gate + nb0 + 8 * rc + 4);
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const int64_t m = mb0 + 8 * k + lane / 8;
            const int64_t mm = m < p.M ? m : 0;  // rows past M read row 0 and are not stored
            old[k] = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(p.out) + mm * p.ldo + nb0 + 8 * rc);
        }
    }

    // ---- low-rank branch: acc += pu[n] . bf16(lora[m]) over r = 0..31, two 32x32x16 bf16 MFMAs per subtile
    if (p.lora) {
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                bf16x8 lb;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    lb[e] = __builtin_bit_cast(__bf16, f32_to_bf16(lr[j][h][0][e]));
                    lb[4 + e] = __builtin_bit_cast(__bf16, f32_to_bf16(lr[j][h][1][e]));
                }
#pragma unroll
                for (int i = 0; i < TN; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[i][h], lb, acc[i][j], 0, 0, 0);
            }
    }

    // ---- bias, activation, bf16, into the staging rows (token j * 32 + lane % 32, feature i * 32 + 8 q + 4 half)
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const uint16_t bv[4] = {uint16_t(bias[i][q].x), uint16_t(bias[i][q].x >> 16), uint16_t(bias[i][q].y),
                                        uint16_t(bias[i][q].y >> 16)};
                uint16_t r[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float y = acc[i][j][4 * q + e];
                    y = y + bf16_to_f32(bv[e]);  // -0 without a bias
                    r[e] = f32_to_bf16(EPI == EPI_GELU ? gelu_tanh(y) : y);
                }
                *reinterpret_cast<uint2*>(stage + (j * 32 + lane % 32) * STG + i * 32 + 8 * q + 4 * half) =
                    make_uint2(r[0] | (uint32_t(r[1]) << 16), r[2] | (uint32_t(r[3]) << 16));
            }
    asm volatile("" ::: "memory");  // the staging writes stay ahead of the reads (one wave: LDS keeps its order)

    // ---- token-major: out[m][nb0 + 8 rc ..] for m = mb0 + 8 k + lane / 8
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int ml = 8 * k + lane / 8;
        const int64_t m = mb0 + ml;
        const uint16_t* sr = stage + ml * STG + 8 * rc;
        const uint2 a0 = *reinterpret_cast<const uint2*>(sr), a1 = *reinterpret_cast<const uint2*>(sr + 4);
        uint4 w = make_uint4(a0.x, a0.y, a1.x, a1.y);
        if (EPI == EPI_RESIDUAL) {
            const uint32_t yw[4] = {w.x, w.y, w.z, w.w}, ow[4] = {old[k].x, old[k].y, old[k].z, old[k].w};
            const float g[8] = {gate[0].x, gate[0].y, gate[0].z, gate[0].w, gate[1].x, gate[1].y, gate[1].z, gate[1].w};
            uint32_t rw[4];
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                const float y0 = bf16_to_f32(uint16_t(yw[d])), y1 = bf16_to_f32(uint16_t(yw[d] >> 16));
                const float o0 = bf16_to_f32(uint16_t(ow[d])), o1 = bf16_to_f32(uint16_t(ow[d] >> 16));
                rw[d] = f32_to_bf16(o0 + y0 * g[2 * d]) | (uint32_t(f32_to_bf16(o1 + y1 * g[2 * d + 1])) << 16);
            }
            w = make_uint4(rw[0], rw[1], rw[2], rw[3]);
            if (p.lnp) {  // this token's chunk (nb0 + 8 rc) / 32: lanes rc % 4 = 0..3 hold its quads 0-1 .. 6-7
                const uint32_t ww[4] = {w.x, w.y, w.z, w.w};
                float v[8];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    v[2 * d] = bf16_to_f32(uint16_t(ww[d]));
                    v[2 * d + 1] = bf16_to_f32(uint16_t(ww[d] >> 16));
                }
                float S = quad_sum(v[0], v[1], v[2], v[3]) + quad_sum(v[4], v[5], v[6], v[7]);
                S = xor_sum<2>(xor_sum<1>(S));
                const float mc = S * (1.0f / 32);
                float M2 = quad_sq(v[0], v[1], v[2], v[3], mc) + quad_sq(v[4], v[5], v[6], v[7], mc);
                M2 = xor_sum<2>(xor_sum<1>(M2));
                if (rc % 4 == 0 && m < p.M) p.lnp[m * (p.N / 32) + (nb0 + 8 * rc) / 32] = make_float2(S, M2);
            }
        }
        if (m < p.M) *reinterpret_cast<uint4*>(static_cast<uint16_t*>(p.out) + m * p.ldo + nb0 + 8 * rc) = w;
    }
}

// Epilogue of the fused GELU MLP's first GEMM (Nunchaku's fused_gelu_mlp, as live::w4a4_gelu_mlp runs it:
// native/ops/w4a4_ops.cpp:42-63; quantization/w4a4.py:195-204), for a wave's 64 x 64 subtile of a 128 x 128 tile:
//   y  = the group sums + bf16(lora[m]) . pu[n] + bias[n]        (as the plain epilogue)
//   h  = GELU_tanh(y) in fp32 (never stored)
//   u  = (h + 0.171875) / smooth2[n] (IEEE quotient); per token and 64-feature group: scale = bf16(max|u| / 15),
//        q = clamp(rint(u / scale), 0, 15) -> the second GEMM's activation codes and scales;
//   lora2 partial = h . proj_down2 over the tile's 128 features, into lpart[tile][m] (a second launch adds the
//        tiles in order).
// The wave's 64 features are one 64-group, so lane (token, half) holds 32 of the group's features (rows
// 32 ti + 8 q + 4 half + e) and the group maximum is one exchange with lane ^ 32. One v_permlane32_swap per value
// pair then gives each lane the 32 features of its own half of the group in order (positions 8 q + e from the
// first result, 8 q + 4 + e from the second), which one hardware fp6 conversion packs. The low-rank product uses
// h split exactly into bf16 hi + lo parts (two MFMAs per 16 features, about 16 significant bits of h) with the
// k-slots of both operands mapped to the features the lane already holds. Rows m >= M get zero codes, scales and
// partials.
// div_rn for w > 0 or w = +0, whose quotient needs no sign fix-up: here u = (GELU(y) + 0.171875) / s with GELU
// above -0.1700, and u / scale with u > 0 (with r = 0 the result is +0)
__device__ __forceinline__ float div_rn_pos(float w, float d, float r) {
    const float q0 = w * r;
    return fmaf(fmaf(-q0, d, w), r, q0);
}

template <int TN, int TM>
__device__ __forceinline__ void finish_tile_gelu_quant(const GemmArgs& p, f32x16 (&acc)[TN][TM], int64_t nb0,
                                                       int64_t mb0, int wn, int wm, int lane, float* xch) {
    static_assert(TN == 2 && TM == 2, "64 x 64 per wave: one 64-feature group");
    const int half = lane / 32, tok = lane % 32;
    const int64_t N = p.N;
    // ---- loads: this layer's low-rank operands and bias, smooth2 and proj_down2^T for the lane's features
    bf16x8 pa[TN][2];
    float4 lr[TM][2][2];
    if (p.lora) {
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int h = 0; h < 2; ++h)
                pa[i][h] = *reinterpret_cast<const bf16x8*>(p.pu + (nb0 + i * 32 + tok) * 32 + h * 16 + 8 * half);
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const float* l = p.lora + (mb0 + j * 32 + tok) * 32 + h * 16 + 8 * half;
                lr[j][h][0] = *reinterpret_cast<const float4*>(l);
                lr[j][h][1] = *reinterpret_cast<const float4*>(l + 4);
            }
    }
    uint2 pdv[TN][2][2];  // proj_down2^T row tok: features 32 ti + 16 qp + 8 part + 4 half .. + 3
#pragma unroll
    for (int i = 0; i < TN; ++i) {
#pragma unroll
        for (int qp = 0; qp < 2; ++qp)
#pragma unroll
            for (int part = 0; part < 2; ++part)
                pdv[i][qp][part] = *reinterpret_cast<const uint2*>(p.pd2t + int64_t(tok) * N + nb0 + i * 32 + 16 * qp +
                                                                  8 * part + 4 * half);
    }

    // ---- this layer's low-rank term, then h = GELU(y + bias) in place
    if (p.lora) {
#pragma unroll
        for (int j = 0; j < TM; ++j)
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                bf16x8 lb;
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    lb[e] = __builtin_bit_cast(__bf16, f32_to_bf16(lr[j][h][0][e]));
                    lb[4 + e] = __builtin_bit_cast(__bf16, f32_to_bf16(lr[j][h][1][e]));
                }
#pragma unroll
                for (int i = 0; i < TN; ++i) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa[i][h], lb, acc[i][j], 0, 0, 0);
            }
    }
    // smooth2, its IEEE reciprocal and the bias (fp32; -0 when absent, an exact identity of the sum) at the lane's
    // 32 features: lane l loads and divides once, for the wave's feature nb0 + l, into the wave's 768-byte LDS slot
    // past the exchange area ([64 reciprocals][64 smooth2][64 bias]), and reads back the 32 it needs (the 32 lanes
    // of a half need the same ones; one wave's LDS accesses complete in order)
    float* const rslot = xch + 4 * TM * 16 * 64 + (wm * 2 + wn) * 192;
    {
        const float sv = bf16_to_f32(p.sm2[nb0 + lane]);
        rslot[lane] = 1.0f / sv;
        rslot[64 + lane] = sv;
        rslot[128 + lane] = p.bias ? bf16_to_f32(p.bias[nb0 + lane]) : -0.0f;
    }
    asm volatile("" ::: "memory");
    float rsm[TN][16], smf[TN][16], bsf[TN][16];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 r4 = *reinterpret_cast<const float4*>(rslot + i * 32 + 8 * q + 4 * half);
            const float4 s4 = *reinterpret_cast<const float4*>(rslot + 64 + i * 32 + 8 * q + 4 * half);
            const float4 b4 = *reinterpret_cast<const float4*>(rslot + 128 + i * 32 + 8 * q + 4 * half);
            rsm[i][4 * q] = r4.x;
            rsm[i][4 * q + 1] = r4.y;
            rsm[i][4 * q + 2] = r4.z;
            rsm[i][4 * q + 3] = r4.w;
            smf[i][4 * q] = s4.x;
            smf[i][4 * q + 1] = s4.y;
            smf[i][4 * q + 2] = s4.z;
            smf[i][4 * q + 3] = s4.w;
            bsf[i][4 * q] = b4.x;
            bsf[i][4 * q + 1] = b4.y;
            bsf[i][4 * q + 2] = b4.z;
            bsf[i][4 * q + 3] = b4.w;
        }
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int k = 0; k < 16; ++k)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j][k] = gelu_tanh(acc[i][j][k] + bsf[i][k]);

    const int64_t g = nb0 / 64;  // the group of the second layer's input
    float* mine = xch + (wm * 2 + wn) * TM * 16 * 64;  // this wave's low-rank partials, lane-linear
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int64_t m = mb0 + j * 32 + tok;
        const bool live = m < p.M;
        // ---- second layer's low-rank down projection: la[r][m] = sum over the 64 features of pd2[n][r] h[m][n]
        f32x16 la = {};
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int qp = 0; qp < 2; ++qp) {
                bf16x8 hi, lo;
#pragma unroll
                for (int t = 0; t < 8; ++t) {
                    const float v = acc[i][j][4 * (2 * qp + t / 4) + t % 4];
                    const uint16_t b = f32_to_bf16(v);
                    hi[t] = __builtin_bit_cast(__bf16, b);
                    lo[t] = __builtin_bit_cast(__bf16, f32_to_bf16(v - bf16_to_f32(b)));
                }
                const bf16x8 a = __builtin_bit_cast(bf16x8, make_uint4(pdv[i][qp][0].x, pdv[i][qp][0].y,
                                                                        pdv[i][qp][1].x, pdv[i][qp][1].y));
                la = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, hi, la, 0, 0, 0);
                la = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, lo, la, 0, 0, 0);
            }
#pragma unroll
        for (int i = 0; i < 16; ++i) mine[(j * 16 + i) * 64 + lane] = live ? la[i] : 0.0f;

        // ---- unsigned int4 quantization of (h + shift) / smooth2 over the token's 64-feature group
        float u[TN][16];
        float amax = 0.0f;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int k = 0; k < 16; ++k) {
                u[i][k] = div_rn_pos(acc[i][j][k] + GELU_SHIFT, smf[i][k], rsm[i][k]);
                amax = fmaxf(amax, fabsf(u[i][k]));
            }
        amax = xor_max<32>(amax);  // the group's other 32 features
        const uint16_t sb = f32_to_bf16(amax / 15.0f);
        const float sc = bf16_to_f32(sb);
        // a row past M (or a group of zeros) takes a zero reciprocal: every quotient below is then +0, code 0
        const float rsc = live && sc > 0.0f ? 1.0f / sc : 0.0f;
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int k = 0; k < 16; ++k)  // u becomes q / 2 (an fp6 e2m3 value) of feature 32 i + 8 (k / 4) + 4 half + k % 4
                u[i][k] = fminf(__builtin_rintf(div_rn_pos(u[i][k], sc, rsc)), 15.0f) * 0.5f;
        // lanes l and l + 32 trade: afterwards the first result holds feature 32 half + 8 q + e of the group and
        // the second 32 half + 8 q + 4 + e (the swap exchanges the upper 32 lanes of its first operand with the
        // lower 32 lanes of its second)
        f32x16 ea, eb;  // even / odd positions of the lane's half (the conversion interleaves its operands)
#pragma unroll
        for (int k = 0; k < 16; ++k) {
            const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(u[0][k]), __float_as_uint(u[1][k]), false,
                                                            false);
            const int q = k / 4, e = k % 4;
            const int p0 = 8 * q + e, p1 = 8 * q + 4 + e;
            if (p0 % 2 == 0) ea[p0 / 2] = __uint_as_float(r[0]);
            else eb[p0 / 2] = __uint_as_float(r[0]);
            if (p1 % 2 == 0) ea[p1 / 2] = __uint_as_float(r[1]);
            else eb[p1 / 2] = __uint_as_float(r[1]);
        }
        u32x6 w;
        asm volatile("v_cvt_scalef32_2xpk16_fp6_f32 %0, %1, %2, 1.0" : "=&v"(w) : "v"(ea), "v"(eb));
        uint8_t* dst = p.q2 + blocked6_offset(m, g, N);
        *reinterpret_cast<uint4*>(dst + 16 * half) = make_uint4(w[0], w[1], w[2], w[3]);
        *reinterpret_cast<uint2*>(dst + 32 + 8 * half) = make_uint2(w[4], w[5]);
        if (half == 0) p.as2[g * p.Mp + m] = live ? sb : uint16_t(0);
    }

    // ---- the tile's two 64-feature halves (waves wn = 0, 1 of a token row) added in that order
    __syncthreads();
    if (wn == 0) {
        const float* other = xch + (wm * 2 + 1) * TM * 16 * 64;
        const int64_t tile = nb0 / 128;
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const int64_t m = mb0 + j * 32 + tok;
            float* dst = p.lpart + (tile * p.Mp + m) * 32 + 4 * half;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int i = (j * 16 + 4 * q + e) * 64 + lane;
                    v[e] = mine[i] + other[i];
                }
                *reinterpret_cast<float4*>(dst + 8 * q) = make_float4(v[0], v[1], v[2], v[3]);
            }
        }
    }
}

// The main loop of both GEMMs. W4: the W4A4 product (fp6 tile-blocked codes, per-group scale fold, scales
// streamed with the codes); otherwise the FP8 product (e4m3 row-major codes only, one fp32 accumulation over all
// of K in the MFMA accumulator).
// One 32 x 32 piece (features n0 .., tokens m0 ..) summed over all of K by NWT waves: wave v folds the 64-deep
// groups [v G / NWT, (v + 1) G / NWT) in increasing order with the tiles' arithmetic (the fp6 product, the exact
// scale product of a bf16 MFMA, one fmaf per element and group), in batches of at most PD groups. load() reads a
// batch's operands straight from global memory into registers (the rows as the tiles read them: 16 + 8 bytes of
// a 48-byte row per lane; lanes 32..63 give the zero k-slots of the scale product); fold() continues the wave's
// partial sums in the MFMA layout with the batch's groups.
template <int NWT, int PD>
struct Piece {
    u32x6 fa[PD], fb[PD];  // the 6 code dwords of each operand row (the MFMA's 8-dword operand gets 2 zeros)
    uint32_t sa[PD], sb[PD];
    int n;  // groups of this batch (wave-uniform)

    // the groups [gb, gb + cnt) of wave v's range (cnt <= PD; cnt = 0 loads a valid dummy and folds nothing)
    __device__ __forceinline__ void load(const GemmArgs& p, int64_t n0, int64_t m0, int gb, int cnt, int lane) {
        const int64_t G = p.K / 64;
        n = cnt;
        const int half = lane / 32;
        const int64_t nr = n0 + lane % 32, mr = m0 + lane % 32;
        const uint8_t* arow = p.wc + (nr / BLOCK_ROWS) * G * BLOCK6 + (nr % BLOCK_ROWS) * ROW6;
        const uint8_t* brow = p.qa + (mr / BLOCK_ROWS) * G * BLOCK6 + (mr % BLOCK_ROWS) * ROW6;
        const int q0 = 16 * half, q1 = 32 + 8 * half;
        const bool low = lane < 32;
#pragma unroll
        for (int d = 0; d < PD; ++d) {
            const int64_t gg = n > 0 ? gb + (d < n ? d : n - 1) : 0;  // in range; groups d >= n are not folded
            const uint4 xa = *reinterpret_cast<const uint4*>(arow + gg * BLOCK6 + q0);
            const uint2 ya = *reinterpret_cast<const uint2*>(arow + gg * BLOCK6 + q1);
            const uint4 xb = *reinterpret_cast<const uint4*>(brow + gg * BLOCK6 + q0);
            const uint2 yb = *reinterpret_cast<const uint2*>(brow + gg * BLOCK6 + q1);
            fa[d] = u32x6{xa.x, xa.y, xa.z, xa.w, ya.x, ya.y};
            fb[d] = u32x6{xb.x, xb.y, xb.z, xb.w, yb.x, yb.y};
            const uint32_t w = p.ws[gg * p.N + nr];
            const uint32_t a = p.as[gg * p.Mp + mr];
            sa[d] = low ? w : 0u;
            sb[d] = low ? a : 0u;
        }
    }

    __device__ __forceinline__ f32x16 fold(f32x16 acc) const {
        const f32x16 zero = {};
#pragma unroll
        for (int d = 0; d < PD; ++d) {
            if (d < n) {
                const i16x4 oa = __builtin_bit_cast(i16x4, make_uint2(sa[d], 0u));
                const i16x4 ob = __builtin_bit_cast(i16x4, make_uint2(sb[d] * 0x10001u, 0u));
                const i32x8 a = {int(fa[d][0]), int(fa[d][1]), int(fa[d][2]), int(fa[d][3]), int(fa[d][4]),
                                 int(fa[d][5]), 0, 0};
                const i32x8 b = {int(fb[d][0]), int(fb[d][1]), int(fb[d][2]), int(fb[d][3]), int(fb[d][4]),
                                 int(fb[d][5]), 0, 0};
                const f32x16 I = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a, b, zero, 3, 2, 0, 0, 0, 0);
                const f32x16 P = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(oa, ob, zero, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[e] = fmaf(I[e], P[e], acc[e]);
            }
        }
        return acc;
    }
};
// a piece: 8 waves, each folding its share of K in batches of 6 groups (one batch up to K = 48 groups), at most
// 5 batches (K up to 240 groups)
constexpr int PIECE_WAVES = 8, PIECE_GROUPS = 6, PIECE_BATCHES = 5;

// How a launch covers the tiles: one tile per workgroup, stream-K shares, or the balanced form (one workgroup of
// two K-groups per CU, whole tiles dealt evenly, the leftover tiles in 32 x 32 pieces).
enum Mode { MODE_TILE = 0, MODE_SK = 1, MODE_BAL = 2 };

template <int BN, int BM, int WN, int WM, int NW, int EPI, int STAGES, bool W4, int MODE = MODE_TILE>
__device__ __forceinline__ void gemm_body(const GemmArgs& p) {
    static_assert(!W4 || (BN % BLOCK_ROWS == 0 && BM % BLOCK_ROWS == 0), "blocked operands come in 128-row tiles");
    // K-groups: MODE_BAL runs 2 x NW waves, each group of NW its own ring over half of a tile's K
    constexpr int KS = MODE == MODE_BAL ? 2 : 1;
    static_assert(KS == 1 || (W4 && BN == 128 && BM == 128 && WN == 64 && WM == 64 && NW == 4), "balanced form");
    static_assert((BN / WN) * (BM / WM) == NW, "wave grid");
    static_assert(STAGES >= 4 && STAGES <= 8, "ring depth");
    constexpr int TN = WN / 32, TM = WM / 32;
    // FP8: 16-byte loads per wave per group of activation codes and of weight codes
    constexpr int XI = W4 ? 0 : BM * 4 / 64 / NW;
    constexpr int WI = W4 ? 0 : BN * 4 / 64 / NW;
    static_assert(W4 || (XI >= 1 && WI >= 1 && BM * 4 == XI * 64 * NW && BN * 4 == WI * 64 * NW), "tile vs waves");
    // W4A4: a stage's codes ((BN + BM) rows of 48 bytes) in CB bytes per wave: N16 16-byte and N4 4-byte loads
    constexpr int CS = (BN + BM) * ROW6, CB = CS / NW;
    constexpr int N16 = W4 ? CB / 1024 : 0, N4 = W4 ? CB % 1024 / 256 : 0;
    static_assert(!W4 || (CS % NW == 0 && CB % 256 == 0), "fp6 stage vs waves");
    // W4: SL 4-byte loads of scales per wave (256 bytes each): ws[BN] pairs, as[BM], then padding
    constexpr int SL = W4 ? (4 * BN + 2 * BM + NW * 256 - 1) / (NW * 256) : 0;
    constexpr int LPG = W4 ? N16 + N4 + SL : XI + WI;  // loads per wave per group
    constexpr int SD = NW * 256 * (SL > 1 ? SL : 1);   // scale bytes loaded per stage
    constexpr int SB = SD + 256;           // + 128 zero bytes (rounded up) read by lanes 32..63
    static_assert(!W4 || 4 * BN + 2 * BM <= SD, "scale stage");
    __shared__ __attribute__((aligned(1024))) uint8_t sX[W4 ? 1 : STAGES][W4 ? 16 : BM * 64];
    __shared__ __attribute__((aligned(1024))) uint8_t sW[W4 ? 1 : STAGES][W4 ? 16 : BN * 64];
    __shared__ __attribute__((aligned(1024))) uint8_t sC[W4 ? KS * STAGES : 1][W4 ? CS : 16];
    __shared__ __attribute__((aligned(256))) uint8_t sS[W4 ? KS * STAGES : 1][W4 ? SB : 256];
    // MODE_BAL: a piece's partial sums, apart from the rings
    __shared__ __attribute__((aligned(16))) uint8_t sE[KS == 2 ? PIECE_WAVES * 64 * 16 * 4 : 16];
    static_assert(KS == 1 || (KS * NW == PIECE_WAVES && NW * 64 * 64 * 4 <= KS * STAGES * CS &&
                              NW * 64 * STG * 2 <= STAGES * CS),
                  "a K-group's accumulators fit the rings, its staging its own ring");

    const int t = threadIdx.x, lane = t % 64;
    const int wall = __builtin_amdgcn_readfirstlane(t / 64);
    const int kg = KS == 1 ? 0 : wall / NW;        // K-group
    const int wave = KS == 1 ? wall : wall % NW;   // wave within the K-group
    const int wn = wave % (BN / WN), wm = wave / (BN / WN);
    const int64_t ntn = p.N / BN, ntm = p.Mp / BM, total = ntn * ntm;
    const int64_t K = p.K, G = K / 64;
    uint8_t* const C0 = &sC[0][0] + (W4 ? kg * (STAGES * CS) : 0);  // this K-group's ring
    uint8_t* const S0 = &sS[0][0] + (W4 ? kg * (STAGES * SB) : 0);

    // zero tails of the scale stages (written once; the loads never touch them)
    if constexpr (W4)
        if (t < KS * STAGES * 32) *reinterpret_cast<uint32_t*>(&sS[t / 32][SD + (t % 32) * 4]) = 0u;

    // per-lane LDS offsets (stage-independent). W4: a lane's 16-byte and 8-byte pieces of its operand row, the
    // scale entries. FP8: operand rows and the two swizzled quarters.
    const bool low = lane < 32;
    const int half = lane / 32;
    int aoff[TN], soa[TN], boff[TM], sob[TM];
    int q0, q1;
#pragma unroll
    for (int i = 0; i < TN; ++i) {
        const int row = wn * WN + i * 32 + lane % 32;
        aoff[i] = W4 ? row * ROW6 : row * 64;
        soa[i] = low ? 4 * row : SD + 4 * (lane % 32);
    }
#pragma unroll
    for (int j = 0; j < TM; ++j) {
        const int row = wm * WM + j * 32 + lane % 32;
        boff[j] = W4 ? (BN + row) * ROW6 : row * 64;
        sob[j] = low ? 4 * BN + 2 * row : SD + 2 * (lane % 32);
    }
    if constexpr (W4) {
        q0 = 16 * half;      // bytes 0..15 of the lane's half
        q1 = 32 + 8 * half;  // bytes 16..23
    } else {
        // every operand row index here is 32-aligned plus lane % 32, so (row / 4) % 4 = (lane % 32 / 4) % 4
        const int sw = ((lane % 32) >> 2) & 3;
        q0 = ((2 * half) ^ sw) * 16;
        q1 = ((2 * half + 1) ^ sw) * 16;
    }
    static_assert(WN % 32 == 0 && WM % 32 == 0, "32-aligned subtiles");

    f32x16 acc[TN][TM];
    // Multiply groups [g0, g1) of the tile at features n0, tokens m0 into acc (zeroed first); on return every load
    // of the piece has landed.
    auto mainloop = [&](int64_t n0, int64_t m0, int g0, int g1) {
        const int GI = g1 - g0;
        // W4: the stage is cut into 1 KB chunks (16-byte loads) and then 256-byte chunks (4-byte loads); wave w takes
        // 1 KB chunks w N16 .. and 256-byte chunks w N4 ... Each chunk lies inside one operand's 6 KB block (block
        // and operand boundaries are multiples of 1 KB), so a load reads from a wave-uniform base (scalar registers:
        // operand, tile row block, chunk; group g adds g BLOCK6) plus lane * 16 or lane * 4. The scale chunk of wave w
        // is bytes 256 w .. of [ws[BN] pairs | as[BM] | padding], also uniform per wave (4 BN and 2 BM are multiples
        // of 256).
        // FP8: this lane's sources. Both relative to group g0 of the piece.
        const uint8_t* cbase[W4 ? N16 + N4 : 1];
        int cdst[W4 ? N16 + N4 : 1];
        const uint8_t* xsrc[W4 ? 1 : XI];
        const uint8_t* wsrc[W4 ? 1 : WI];
        if constexpr (W4) {
#pragma unroll
            for (int u = 0; u < N16 + N4; ++u) {
                const int o = u < N16 ? (wave * N16 + u) * 1024 : NW * N16 * 1024 + (wave * N4 + u - N16) * 256;
                cdst[u] = o;
                cbase[u] = (o < BN * ROW6 ? p.wc + (n0 / BLOCK_ROWS + o / BLOCK6) * G * BLOCK6 + o % BLOCK6
                                          : p.qa + (m0 / BLOCK_ROWS + (o - BN * ROW6) / BLOCK6) * G * BLOCK6 +
                                                (o - BN * ROW6) % BLOCK6) +
                           int64_t(g0) * BLOCK6;
            }
        } else {
#pragma unroll
            for (int j = 0; j < XI; ++j) {
                const int slot = (wave * XI + j) * 64 + lane;          // 16-byte slot of the stage
                const int row = slot / 4, quarter = (slot % 4) ^ ((row >> 2) & 3);
                xsrc[j] = p.qa + (m0 + row) * K + quarter * 16 + int64_t(g0) * 64;
            }
#pragma unroll
            for (int j = 0; j < WI; ++j) {
                const int slot = (wave * WI + j) * 64 + lane;
                const int row = slot / 4, quarter = (slot % 4) ^ ((row >> 2) & 3);
                wsrc[j] = p.wc + (n0 + row) * K + quarter * 16 + int64_t(g0) * 64;
            }
        }
        // the wave's SL chunks of 256 scale bytes of group g0 (chunk c = wave SL + u at byte 256 c of the stage): ws,
        // as or (padding) a valid dummy
        const uint8_t* sbase[SL > 0 ? SL : 1];
        int64_t sstride[SL > 0 ? SL : 1];
#pragma unroll
        for (int u = 0; u < SL; ++u) {
            const int b = 256 * (wave * SL + u);
            if (b < 4 * BN) {
                sstride[u] = 4 * p.N;
                sbase[u] = reinterpret_cast<const uint8_t*>(p.ws + n0) + b + g0 * sstride[u];
            } else if (b < 4 * BN + 2 * BM) {
                sstride[u] = 2 * p.Mp;
                sbase[u] = reinterpret_cast<const uint8_t*>(p.as + m0) + (b - 4 * BN) + g0 * sstride[u];
            } else {
                sbase[u] = reinterpret_cast<const uint8_t*>(p.ws + n0);
                sstride[u] = 0;
            }
        }
        const uint32_t off16 = uint32_t(lane) * 16, off4 = uint32_t(lane) * 4;

        // direct load u (0 .. LPG - 1) of group g0 + g (clamped to the piece's last group) into stage st
        auto issue_one = [&](int st, int g, int u) {
            const int gg = g < GI ? g : GI - 1;
            if constexpr (W4) {
                if (u < N16) dma16s(cbase[u] + int64_t(gg) * BLOCK6, off16, lds_addr(C0 + st * CS + cdst[u]));
                else if (u < N16 + N4) dma4s(cbase[u] + int64_t(gg) * BLOCK6, off4, lds_addr(C0 + st * CS + cdst[u]));
                else dma4s(sbase[u - N16 - N4] + gg * sstride[u - N16 - N4], off4,
                           lds_addr(S0 + st * SB + (wave * SL + u - N16 - N4) * 256));
            } else {
                if (u < XI) dma16(xsrc[u] + int64_t(gg) * 64, lds_addr(&sX[st][(wave * XI + u) * 1024]));
                else dma16(wsrc[u - XI] + int64_t(gg) * 64, lds_addr(&sW[st][(wave * WI + u - XI) * 1024]));
            }
        };

        const f32x16 zero = {};

        // Two register sets of one group's operands: weight / activation code fragments (W4: 6 dwords of fp6 codes,
        // FP8: 8 of e4m3) and (W4) the scales of each fragment row: the weight scale's bf16 pair, the activation
        // scale zero-extended (lanes 32..63 read the zero tail).
        // Group h is multiplied from set h % 2 while group h + 1 is read into the other set.
        i32x8 fa[2][TN], fb[2][TM];
        uint32_t fsa[2][TN], fsb[2][TM];
        auto load_frag = [&](const uint8_t* r) {
            if constexpr (W4) {
                const uint4 x = *reinterpret_cast<const uint4*>(r + q0);
                const uint2 y = *reinterpret_cast<const uint2*>(r + q1);
                return i32x8{int(x.x), int(x.y), int(x.z), int(x.w), int(y.x), int(y.y), 0, 0};
            } else {
                const uint4 x = *reinterpret_cast<const uint4*>(r + q0), y = *reinterpret_cast<const uint4*>(r + q1);
                return i32x8{int(x.x), int(x.y), int(x.z), int(x.w), int(y.x), int(y.y), int(y.z), int(y.w)};
            }
        };
        auto load_a = [&](int set, int st, int i) {
            if constexpr (W4) {
                fa[set][i] = load_frag(C0 + st * CS + aoff[i]);
                fsa[set][i] = *reinterpret_cast<const uint32_t*>(S0 + st * SB + soa[i]);
            } else {
                fa[set][i] = load_frag(&sW[st][aoff[i]]);
            }
        };
        auto load_b = [&](int set, int st, int j) {
            if constexpr (W4) {
                fb[set][j] = load_frag(C0 + st * CS + boff[j]);
                fsb[set][j] = *reinterpret_cast<const uint16_t*>(S0 + st * SB + sob[j]);
            } else {
                fb[set][j] = load_frag(&sX[st][boff[j]]);
            }
        };
        // fragment r of the next group (r < TN: weight rows i = r, else activation rows j = r - TN)
        auto load_next = [&](int set, int st, int r) {
            if (r < TN) load_a(set, st, r);
            else load_b(set, st, r - TN);
        };

        // Multiply one group from register set cur while the next group's operands (stage nst) are read into the other
        // set, TN + TM fragments spread over the TN x TM subtiles: the reads have a whole step to land, so LDS latency
        // stays off the MFMA chain.
        // W4: the fold is software-pipelined by one subtile: the products of subtile s are folded while the MFMAs of
        // subtile s + 1 run (the last subtile of a group while the first subtile of the next group runs). pI / pP hold
        // the pending subtile; they start at zero (the first fold adds 0 * 0 to a zero accumulator: no change).
        f32x16 pI = zero, pP = zero;
        // The step's LPG direct loads (group ig into stage ist) are spread over its subtiles, one or two after each
        // subtile's MFMAs, so a wave never waits on a full load queue with MFMA work still to issue.
        constexpr int NF = TN + TM, NS = TN * TM;
        auto step = [&](int cur, int nst, int ist, int ig) {
#pragma unroll
            for (int s = 0; s < NS; ++s) {
                const int i = s / TM, j = s % TM;
                if constexpr (W4) {
                    const int pi = s == 0 ? TN - 1 : (s - 1) / TM, pj = s == 0 ? TM - 1 : (s - 1) % TM;
                    // k-slots 0 and 1: (hi, lo) of ws against (as, as)
                    const i16x4 oa = __builtin_bit_cast(i16x4, make_uint2(fsa[cur][i], 0u));
                    const i16x4 ob = __builtin_bit_cast(i16x4, make_uint2(fsb[cur][j] * 0x10001u, 0u));
                    // A: weights as e3m2 (format 3), B: activations as e2m3 (format 2)
                    const f32x16 I =
                        __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[cur][i], fb[cur][j], zero, 3, 2, 0, 0, 0, 0);
                    const f32x16 P = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(oa, ob, zero, 0, 0, 0);
#pragma unroll
                    for (int e = 0; e < 16; ++e) acc[pi][pj][e] = fmaf(pI[e], pP[e], acc[pi][pj][e]);
                    pI = I;
                    pP = P;
                } else {
                    acc[i][j] =
                        __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(fa[cur][i], fb[cur][j], acc[i][j], 0, 0, 0, 0, 0, 0);
                }
#pragma unroll
                for (int r = s * NF / NS; r < (s + 1) * NF / NS; ++r) load_next(1 - cur, nst, r);
                // one wave issues in order and an MFMA waits at issue while the matrix core is busy, so the fold of
                // subtile s - 1 is split around the two MFMAs of subtile s: it executes while they run
                if constexpr (W4) {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // I_s (32 cycles)
                    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);   // reads of the next group
                    __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);  // fold of s - 1, first part
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);   // P_s (32 cycles)
                    __builtin_amdgcn_sched_group_barrier(0x002, 10, 0);  // the rest
                } else {
                    __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
                }
#pragma unroll
                for (int u = s * LPG / NS; u < (s + 1) * LPG / NS; ++u) issue_one(ist, ig, u);
            }
        };

        // Ring, one group per step. Step h: this wave's loads of group h + 1 have landed (the STAGES - 3 groups after
        // it may still be in flight); after the barrier the same holds for every wave, and group h + 1 is read into
        // registers during the step. The stage of group h - 1 is free: every wave read it during step h - 2 and used
        // the registers in step h - 1, so no wait on LDS reads comes before the barrier. Group h + STAGES - 1 goes into
        // it (clamped to the last group, so every step issues the same loads and vmcnt counts stay exact). Stages and
        // register sets are compile-time constants throughout: whole turns of the ring are unrolled, and so are the
        // G % STAGES remaining steps (each under a uniform branch); STAGES is even, so group h uses set h % 2.
        static_assert(STAGES >= 4 && STAGES % 2 == 0, "the ring keeps one stage being read, one free and two or more in "
                                                      "flight; register sets alternate over a turn");
#pragma unroll
        for (int k = 0; k < STAGES - 1; ++k)
#pragma unroll
            for (int u = 0; u < LPG; ++u) issue_one(k, k, u);
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) acc[i][j] = zero;
        wait_vmcnt<(STAGES - 2) * LPG>();
        __syncthreads();
#pragma unroll
        for (int r = 0; r < NF; ++r) load_next(0, 0, r);
        auto ring_step = [&](int k, int h) {
            wait_vmcnt<(STAGES - 3) * LPG>();
            __syncthreads();
            step(k % 2, k + 1 == STAGES ? 0 : k + 1, k == 0 ? STAGES - 1 : k - 1, h + STAGES - 1);
        };
        int g = 0;  // wave-uniform: kept in scalar registers
        for (; g + STAGES <= GI; g = __builtin_amdgcn_readfirstlane(g + STAGES)) {
#pragma unroll
            for (int k = 0; k < STAGES; ++k) ring_step(k, g + k);
        }
#pragma unroll
        for (int k = 0; k < STAGES - 1; ++k)
            if (g + k < GI) ring_step(k, g + k);
        if constexpr (W4) {
#pragma unroll
            for (int e = 0; e < 16; ++e) acc[TN - 1][TM - 1][e] = fmaf(pI[e], pP[e], acc[TN - 1][TM - 1][e]);
        }
        wait_vmcnt<0>();  // the clamped tail loads land before the workgroup can end
    };

    if constexpr (MODE == MODE_TILE) {
        // the whole tile `pid`, ids remapped so that the tiles of one weight slab run on one XCD
        const int64_t pid = blockIdx.x;
        int64_t tile = pid;
        if (total % 8 == 0) tile = (pid % 8) * (total / 8) + pid / 8;
        const int64_t n0 = (tile / ntm) * BN, m0 = (tile % ntm) * BM;
        mainloop(n0, m0, 0, int(G));
        if constexpr (EPI == EPI_GELU_QUANT) {
            static_assert(W4 && BN == 128 && BM == 128 && NW == 4, "the fused GELU epilogue runs on 128 x 128 tiles");
            __syncthreads();  // every wave is past its last read of the ring, whose LDS the exchange reuses
            static_assert((4 * 2 * 16 * 64 + 4 * 192) * 4 <= STAGES * CS, "exchange and per-feature slots fit in the ring");
            finish_tile_gelu_quant<TN, TM>(p, acc, n0 + wn * WN, m0 + wm * WM, wn, wm, lane,
                                           reinterpret_cast<float*>(&sC[0][0]));
        } else if constexpr (W4 && EPI != EPI_F32 && TN == 2 && TM == 2) {
            __syncthreads();  // every wave is past its last read of the ring, whose LDS the staging reuses
            static_assert(NW * 64 * STG * 2 <= STAGES * CS, "staging fits in the ring");
            finish_tile_rows<TN, TM, EPI>(p, acc, n0 + wn * WN, m0 + wm * WM, lane,
                                          reinterpret_cast<uint16_t*>(&sC[0][0]) + wave * 64 * STG);
        } else {
            finish_tile<TN, TM, EPI>(p, acc, n0 + wn * WN, m0 + wm * WM, lane);
        }
    } else if constexpr (MODE == MODE_SK) {
        // Stream-K share of this workgroup: the U = total * G (tile, group) iterations in tile-major order split
        // evenly over the W workgroups of the launch, W > total, so a share covers less than one tile: at most two
        // pieces, whose partial sums go to workspace slots 2 c and 2 c + 1 (c: the logical index, workgroup ids
        // remapped so that consecutive shares run on one XCD); w4a4_merge_kernel adds them per tile and finishes.
        const int64_t W = gridDim.x, U = total * G, pid = blockIdx.x;
        const int64_t c = W % 8 == 0 ? (pid % 8) * (W / 8) + pid / 8 : pid;
        const int64_t s0 = c * U / W, s1 = (c + 1) * U / W;
#pragma unroll 1
        for (int piece = 0; piece < 2; ++piece) {
            const int64_t a0 = piece == 0 ? s0 : (s0 / G + 1) * G;
            if (a0 >= s1) break;
            const int64_t tl = a0 / G;
            const int g0 = int(a0 - tl * G), g1 = int(s1 - tl * G < G ? s1 - tl * G : G);
            if (piece == 1) __syncthreads();  // every wave is past the first piece's ring before the refill
            mainloop((tl / ntm) * BN, (tl % ntm) * BM, g0, g1);
            float4* dst = reinterpret_cast<float4*>(p.part + (2 * c + piece) * (NW * 64 * TN * TM * 16)) +
                          wave * (TN * TM * 4 * 64) + lane;
#pragma unroll
            for (int i = 0; i < TN; ++i)
#pragma unroll
                for (int j = 0; j < TM; ++j)
#pragma unroll
                    for (int f4 = 0; f4 < 4; ++f4)
                        dst[((i * TM + j) * 4 + f4) * 64] = make_float4(acc[i][j][4 * f4], acc[i][j][4 * f4 + 1],
                                                                        acc[i][j][4 * f4 + 2], acc[i][j][4 * f4 + 3]);
        }
    } else {
        // Balanced form: one workgroup per CU (W = gridDim.x, a multiple of 8). The T = total tiles of 128 x 128 are
        // dealt out as F = T / W whole tiles per workgroup; the L = T - F W left over are cut into 16 L <= W pieces
        // of 32 x 32, piece c going to workgroup c. A whole tile is summed by the two K-groups, group 0 over the
        // first half of the groups and group 1 over the second (G is even), added in that order. A piece is summed
        // over all of K by the 8 waves first, each folding an eighth of the groups (at most 6, loaded in one
        // batch); the 8 partial sums wait in LDS, apart from the rings, and wave 0 of K-group 1 adds them in wave
        // order and finishes the piece while K-group 0 finishes the last tile. Results are deterministic; the sums
        // are split in K, so their rounding differs from the one-pass fold as the stream-K launch's does. Tile ids
        // are remapped so that the tiles the workgroups of one XCD (c mod 8) run at the same time are consecutive:
        // a few weight slabs against all row blocks.
        const int64_t W = gridDim.x, c = blockIdx.x, Wx = W / 8;
        const int64_t F = total / W;
        // pieces: P = 16 L of them on workgroups c < P; workgroup c runs on XCD c % 8, so piece pc = (c % 8) P / 8 +
        // c / 8 puts consecutive pieces (the 16 of a leftover tile) on one XCD, whose L2 then holds the tile's
        // operand rows for all of them
        const int64_t P = 16 * (total - F * W);
        const bool piece = c < P;  // workgroup-uniform
        const int64_t pc = (c % 8) * (P / 8) + c / 8;
        const int64_t ptl = F * W + pc / 16;
        const int64_t pn = (ptl / ntm) * BN + 32 * ((pc % 16) / 4), pm = (ptl % ntm) * BM + 32 * (pc % 4);
        float4* const E = reinterpret_cast<float4*>(sE);  // the piece's partial sums, [wave][4][64] float4
        const int hg = int(G / 2);
        float4* const R = reinterpret_cast<float4*>(&sC[0][0]) + wave * (TN * TM * 4 * 64) + lane;
        if (piece) {
            // wave `wall` folds the groups [gb, ge) in batches, the next batch's loads issued before the current
            // batch is folded (two register sets)
            const int gb = int(G * wall / PIECE_WAVES), ge = int(G * (wall + 1) / PIECE_WAVES), ng = ge - gb;
            auto count = [&](int b) {
                const int r = ng - b * PIECE_GROUPS;
                return r < 0 ? 0 : (r < PIECE_GROUPS ? r : PIECE_GROUPS);
            };
            Piece<PIECE_WAVES, PIECE_GROUPS> pa, pb;
            f32x16 part = {};
            pa.load(p, pn, pm, gb, count(0), lane);
            for (int b = 0; b * PIECE_GROUPS < ng; b += 2) {
                const bool more = (b + 1) * PIECE_GROUPS < ng;
                if (more) pb.load(p, pn, pm, gb + (b + 1) * PIECE_GROUPS, count(b + 1), lane);
                part = pa.fold(part);
                if ((b + 2) * PIECE_GROUPS < ng) pa.load(p, pn, pm, gb + (b + 2) * PIECE_GROUPS, count(b + 2), lane);
                if (more) part = pb.fold(part);
            }
#pragma unroll
            for (int f4 = 0; f4 < 4; ++f4)
                E[(wall * 4 + f4) * 64 + lane] =
                    make_float4(part[4 * f4], part[4 * f4 + 1], part[4 * f4 + 2], part[4 * f4 + 3]);
        }
        for (int64_t k = 0; k < F; ++k) {
            const int64_t tile = (c % 8) * (F * Wx) + k * Wx + c / 8;
            const int64_t n0 = (tile / ntm) * BN, m0 = (tile % ntm) * BM;
            if (k > 0) __syncthreads();  // group 0's staging reads are done before its ring is refilled
            mainloop(n0, m0, kg * hg, kg * hg + hg);
            __syncthreads();  // every wave is past its last read of the rings, which now hold group 1's sums
            if (kg == 1)
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
#pragma unroll
                        for (int f4 = 0; f4 < 4; ++f4)
                            R[((i * TM + j) * 4 + f4) * 64] = make_float4(acc[i][j][4 * f4], acc[i][j][4 * f4 + 1],
                                                                          acc[i][j][4 * f4 + 2], acc[i][j][4 * f4 + 3]);
            __syncthreads();
            if (kg == 0)
#pragma unroll
                for (int i = 0; i < TN; ++i)
#pragma unroll
                    for (int j = 0; j < TM; ++j)
#pragma unroll
                        for (int f4 = 0; f4 < 4; ++f4) {
                            const float4 x = R[((i * TM + j) * 4 + f4) * 64];
                            acc[i][j][4 * f4] += x.x;
                            acc[i][j][4 * f4 + 1] += x.y;
                            acc[i][j][4 * f4 + 2] += x.z;
                            acc[i][j][4 * f4 + 3] += x.w;
                        }
            // the sums are read: group 1 may refill its ring, group 0 stages its outputs over its own ring
            __syncthreads();
            if (kg == 0) {
                if constexpr (EPI != EPI_F32)
                    finish_tile_rows<TN, TM, EPI>(p, acc, n0 + wn * WN, m0 + wm * WM, lane,
                                                  reinterpret_cast<uint16_t*>(&sC[0][0]) + wave * 64 * STG);
                else
                    finish_tile<TN, TM, EPI>(p, acc, n0 + wn * WN, m0 + wm * WM, lane);
            }
        }
        if (wall == NW && piece) {  // while group 0 finishes the last tile
            f32x16 part[1][1];
#pragma unroll
            for (int f4 = 0; f4 < 4; ++f4) {
                const float4 x = E[f4 * 64 + lane];
                part[0][0][4 * f4] = x.x;
                part[0][0][4 * f4 + 1] = x.y;
                part[0][0][4 * f4 + 2] = x.z;
                part[0][0][4 * f4 + 3] = x.w;
            }
#pragma unroll
            for (int v = 1; v < PIECE_WAVES; ++v)
#pragma unroll
                for (int f4 = 0; f4 < 4; ++f4) {
                    const float4 x = E[(v * 4 + f4) * 64 + lane];
                    part[0][0][4 * f4] += x.x;
                    part[0][0][4 * f4 + 1] += x.y;
                    part[0][0][4 * f4 + 2] += x.z;
                    part[0][0][4 * f4 + 3] += x.w;
                }
            finish_tile<1, 1, EPI>(p, part, pn, pm, lane);
        }
    }
}

template <int BN, int BM, int WN, int WM, int NW, int EPI, int STAGES>
__global__ __launch_bounds__(NW * 64) void w4a4_gemm_kernel(GemmArgs p) {
    gemm_body<BN, BM, WN, WM, NW, EPI, STAGES, true>(p);
}

template <int EPI, int STAGES>
__global__ __launch_bounds__(512) void w4a4_gemm_bal_kernel(GemmArgs p) {
    gemm_body<128, 128, 64, 64, 4, EPI, STAGES, true, MODE_BAL>(p);
}

template <int BN, int BM, int WN, int WM, int NW, int STAGES>
__global__ __launch_bounds__(NW * 64) void w4a4_gemm_sk_kernel(GemmArgs p) {
    gemm_body<BN, BM, WN, WM, NW, EPI_F32, STAGES, true, MODE_SK>(p);
}

// The stream-K share c (of W) whose iteration range [c U / W, (c + 1) U / W) contains iteration `it`
__device__ __forceinline__ int64_t share_of(int64_t it, int64_t U, int64_t W) {
    int64_t c = it * W / U;
    while (c + 1 < W && (c + 1) * U / W <= it) ++c;
    while (c > 0 && c * U / W > it) --c;
    return c;
}

// One tile of a stream-K launch: the partial sums of its contributors (the shares that meet its G iterations, in
// increasing order, i.e. in increasing K) added in that fixed order into the accumulator layout of the main loop,
// then the low-rank term, bias and epilogue as in the plain launch.
template <int BN, int BM, int WN, int WM, int NW, int EPI>
__global__ __launch_bounds__(NW * 64) void w4a4_merge_kernel(GemmArgs p, int64_t W) {
    constexpr int TN = WN / 32, TM = WM / 32;
    constexpr bool ROWS = EPI == EPI_BF16 || EPI == EPI_RESIDUAL || EPI == EPI_GELU;  // token-major staging
    __shared__ __attribute__((aligned(16))) uint16_t stage[ROWS ? NW * 64 * STG : 8];
    const int t = threadIdx.x, lane = t % 64;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);
    const int wn = wave % (BN / WN), wm = wave / (BN / WN);
    const int64_t ntm = p.Mp / BM, total = (p.N / BN) * ntm, G = p.K / 64, U = total * G;
    const int64_t tl = blockIdx.x;
    const int64_t cf = share_of(tl * G, U, W), cl = share_of((tl + 1) * G - 1, U, W);
    f32x16 acc[TN][TM];
    bool first = true;
    for (int64_t c = cf; c <= cl; ++c) {
        const int64_t cs0 = c * U / W;
        if (cs0 == (c + 1) * U / W) continue;  // an empty share (U < W) wrote nothing
        const int piece = cs0 >= tl * G ? 0 : 1;  // the tile is the first or the second piece of share c
        const float4* src = reinterpret_cast<const float4*>(p.part + (2 * c + piece) * (NW * 64 * TN * TM * 16)) +
                            wave * (TN * TM * 4 * 64) + lane;
        float4 v[TN][TM][4];
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int f4 = 0; f4 < 4; ++f4) v[i][j][f4] = src[((i * TM + j) * 4 + f4) * 64];
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j)
#pragma unroll
                for (int f4 = 0; f4 < 4; ++f4) {
                    const float w4[4] = {v[i][j][f4].x, v[i][j][f4].y, v[i][j][f4].z, v[i][j][f4].w};
#pragma unroll
                    for (int e = 0; e < 4; ++e)
                        acc[i][j][4 * f4 + e] = first ? w4[e] : acc[i][j][4 * f4 + e] + w4[e];
                }
        first = false;
    }
    const int64_t n0 = (tl / ntm) * BN + wn * WN, m0 = (tl % ntm) * BM + wm * WM;
    if constexpr (EPI == EPI_BF16 || EPI == EPI_RESIDUAL || EPI == EPI_GELU)
        finish_tile_rows<TN, TM, EPI>(p, acc, n0, m0, lane, stage + wave * 64 * STG);
    else
        finish_tile<TN, TM, EPI>(p, acc, n0, m0, lane);
}

template <int BN, int BM, int WN, int WM, int NW, int EPI, int STAGES>
__global__ __launch_bounds__(NW * 64) void fp8_gemm_kernel(GemmArgs p) {
    gemm_body<BN, BM, WN, WM, NW, EPI, STAGES, false>(p);
}

// FP8 stream-K shares: the fp32 accumulators of each share's pieces, merged by w4a4_merge_kernel with the FP8
// epilogue
template <int BN, int BM, int WN, int WM, int NW, int STAGES>
__global__ __launch_bounds__(NW * 64) void fp8_gemm_sk_kernel(GemmArgs p) {
    gemm_body<BN, BM, WN, WM, NW, EPI_F32, STAGES, false, MODE_SK>(p);
}

template <int BN, int BM, int WN, int WM, int NW, int ST>
int launch(const GemmArgs& a, int epi, hipStream_t stream) {
    if (a.N % BN || a.Mp % BM) return fail(WDL_EINVAL, "w4a4_gemm: tile %dx%d does not divide N=%lld Mp=%lld", BN, BM,
                                           (long long)a.N, (long long)a.Mp);
    const unsigned grid = unsigned((a.N / BN) * (a.Mp / BM));
    switch (epi) {
        case EPI_BF16: w4a4_gemm_kernel<BN, BM, WN, WM, NW, EPI_BF16, ST><<<grid, NW * 64, 0, stream>>>(a); break;
        case EPI_F32: w4a4_gemm_kernel<BN, BM, WN, WM, NW, EPI_F32, ST><<<grid, NW * 64, 0, stream>>>(a); break;
        case EPI_RESIDUAL: w4a4_gemm_kernel<BN, BM, WN, WM, NW, EPI_RESIDUAL, ST><<<grid, NW * 64, 0, stream>>>(a); break;
        case EPI_GELU: w4a4_gemm_kernel<BN, BM, WN, WM, NW, EPI_GELU, ST><<<grid, NW * 64, 0, stream>>>(a); break;
        default: return fail(WDL_EINVAL, "w4a4_gemm: bad epilogue %d", epi);
    }
    return check_launch("w4a4_gemm");
}

// Tile configuration: 128 x 128 per workgroup (4 waves of 64 x 64, 54 KB of LDS: two workgroups per CU), except
// when those tiles just exceed the CU count (cus < T <= 1.25 cus, e.g. 11 x 24 = 264 at 1392 tokens and
// N = 3072): then 8 CUs would run two tiles and the rest one, and 256 x 128 tiles (8 waves of 64 x 64, 83 KB:
// one per CU, 132 of them) finish sooner (measured: 41.7 -> 38.3 us at K = 3072, 136.6 -> 130.4 us at
// K = 14336). Elsewhere the 128 x 128 tiles are as fast or faster.
//
// Stream-K: when even the 256 x 128 tiles leave a quarter of the CUs or more idle and K is long enough to pay for
// the partial sums (measured: at 1392 tokens, N = 3072, K = 14336, 132 tiles: 113.7 -> 89.9 us; at 2688 tokens,
// 252 tiles on 256 CUs, the partial sums cost 20 us and nothing is gained), one workgroup per CU takes an equal share of the (tile, 64-deep group) iterations and writes
// fp32 partial sums of its (at most two) tile pieces; a second launch adds each tile's pieces in a fixed order and
// applies the epilogue. The sums of a tile are then split in K, so the rounding differs from the one-pass fold
// (the same fp32 fold per piece, then fp32 adds of the pieces): results are deterministic but not bit-identical to
// the plain launch.
#ifndef WDL_GEMM_STAGES
#define WDL_GEMM_STAGES 4
#endif
#ifndef WDL_SK_MIN_GROUPS
#define WDL_SK_MIN_GROUPS 96
#endif
constexpr int SK_NW = 8;                                    // the 256 x 128 configuration
constexpr int64_t SK_SLOT = SK_NW * 64 * 2 * 2 * 16;        // floats per partial: the workgroup's accumulators

// Balanced form (one workgroup of 8 waves per CU: whole 128 x 128 tiles dealt evenly, each summed by two K-groups
// of 4 waves, the leftover tiles in 32 x 32 pieces): when there is at least one tile per CU, the groups split evenly
// in two and either no tile is left over or the pieces come to at most one per CU with K of at most 240 groups (a
// wave's share of a piece in at most 5 batches of loads). It takes the shapes whose tile count just exceeds the CU
// count, where whole-tile launches leave CUs idle: at 1392 tokens, N = 3072 (264 tiles on 256 CUs: o / cross-q /
// cross-o at K = 3072, FFN-down at K = 14336). Measured at K = 3072: the K-split tiles alone 24.0 us against 31.7
// us for the one-pass 256 x 128 launch; the pieces as a separate phase of three memory round trips cost another 5
// us. At K = 14336 it replaces stream-K, whose partial sums and merge launch cost more than the pieces' five
// batches. It needs no memory, but runs (like stream-K) only when the caller passes a workspace: without one every
// shape takes the one-pass fold.
#ifndef WDL_BAL_BATCHES
#define WDL_BAL_BATCHES PIECE_BATCHES
#endif
constexpr int64_t BAL_TOKEN_BYTES = 256;  // the workspace size reported for it
bool bal_fits(int64_t Mp, int64_t N, int64_t K) {
    const int64_t cus = cu_count(), T = (N / 128) * (Mp / 128), G = K / 64;
    if (cus <= 0 || cus % 8 || G % 2 || T < cus) return false;
    return T % cus == 0 || (16 * (T % cus) <= cus && G <= PIECE_WAVES * PIECE_GROUPS * WDL_BAL_BATCHES);
}

// stream-K workgroups for an M x N x K product (0: plain launch)
int64_t sk_shares(int64_t Mp, int64_t N, int64_t K) {
    const int64_t cus = cu_count();
    if (N % 256 || cus <= 0 || K / 64 < WDL_SK_MIN_GROUPS || bal_fits(Mp, N, K)) return 0;
    const int64_t Tw = (N / 256) * (Mp / 128);
    return 4 * Tw <= 3 * cus ? cus : 0;  // the 256 x 128 launch would leave a quarter of the CUs or more idle
}

int dispatch(const GemmArgs& a, int epi, hipStream_t stream) {
    const int64_t T = (a.N / 128) * (a.Mp / 128), cus = cu_count();
    if (a.part && bal_fits(a.Mp, a.N, a.K)) {
        const unsigned grid = unsigned(cus);
        constexpr int ST = WDL_GEMM_STAGES;
        switch (epi) {
            case EPI_BF16: w4a4_gemm_bal_kernel<EPI_BF16, ST><<<grid, 512, 0, stream>>>(a); break;
            case EPI_F32: w4a4_gemm_bal_kernel<EPI_F32, ST><<<grid, 512, 0, stream>>>(a); break;
            case EPI_RESIDUAL: w4a4_gemm_bal_kernel<EPI_RESIDUAL, ST><<<grid, 512, 0, stream>>>(a); break;
            case EPI_GELU: w4a4_gemm_bal_kernel<EPI_GELU, ST><<<grid, 512, 0, stream>>>(a); break;
            default: return fail(WDL_EINVAL, "w4a4_gemm: bad epilogue %d", epi);
        }
        return check_launch("w4a4_gemm balanced");
    }
    const int64_t W = a.part ? sk_shares(a.Mp, a.N, a.K) : 0;
    if (W) {
        const int64_t tiles = (a.N / 256) * (a.Mp / 128);
        w4a4_gemm_sk_kernel<256, 128, 64, 64, SK_NW, WDL_GEMM_STAGES><<<unsigned(W), SK_NW * 64, 0, stream>>>(a);
        int rc = check_launch("w4a4_gemm stream-K");
        if (rc) return rc;
        switch (epi) {
            case EPI_BF16: w4a4_merge_kernel<256, 128, 64, 64, SK_NW, EPI_BF16><<<unsigned(tiles), SK_NW * 64, 0, stream>>>(a, W); break;
            case EPI_F32: w4a4_merge_kernel<256, 128, 64, 64, SK_NW, EPI_F32><<<unsigned(tiles), SK_NW * 64, 0, stream>>>(a, W); break;
            case EPI_RESIDUAL: w4a4_merge_kernel<256, 128, 64, 64, SK_NW, EPI_RESIDUAL><<<unsigned(tiles), SK_NW * 64, 0, stream>>>(a, W); break;
            case EPI_GELU: w4a4_merge_kernel<256, 128, 64, 64, SK_NW, EPI_GELU><<<unsigned(tiles), SK_NW * 64, 0, stream>>>(a, W); break;
            default: return fail(WDL_EINVAL, "w4a4_gemm: bad epilogue %d", epi);
        }
        return check_launch("w4a4_gemm merge");
    }
    if (a.N % 256 == 0 && cus > 0 && T > cus && 4 * T <= 5 * cus)
        return launch<256, 128, 64, 64, 8, WDL_GEMM_STAGES>(a, epi, stream);
    return launch<128, 128, 64, 64, 4, WDL_GEMM_STAGES>(a, epi, stream);
}

// FP8 launches. The fp8 products carry no per-group fold, so the accumulators can take a wave tile of 128 x 64
// (8 subtiles, 128 accumulator registers; the compiler keeps part of the set in AGPRs) with one workgroup of 4 waves
// per CU on a 256 x
// 128 tile, which halves the LDS fragment reads per MFMA of the 64 x 64 wave tile (6 fragments for 8 MFMAs
// against 4 for 4). That wide tile runs whenever N % 256 == 0 and its tiles fill at least 15/16 of the CUs
// (A/B on one box, two runs each, 2640 tokens: QKV 114 -> 106 us, o 39.9 -> 36.9, FFN-up 191 -> 167, FFN-down
// 162 -> 143 us; 1392 tokens: QKV 70.7 -> 67.8 us, FFN-up unchanged); below that (o at 1392 tokens: 132 wide tiles)
// the 128 x 128 tiles of two workgroups per CU keep every CU busy and are faster (29.0 against 31.3 us). Stream-K
// when the caller passes a workspace and the 256 x 128 tiles would leave a quarter of the CUs or more idle with K
// of 96 groups or more (FFN-down at 1392 tokens, K = 14336: 130 -> 101 us).
int64_t fp8_sk_shares(int64_t Mp, int64_t N, int64_t K) {
    const int64_t cus = cu_count();
    if (N % 256 || cus <= 0 || K / 64 < WDL_SK_MIN_GROUPS) return 0;
    return 4 * (N / 256) * (Mp / 128) <= 3 * cus ? cus : 0;
}

template <int EPI>
int launch_fp8_epi(const GemmArgs& a, hipStream_t stream) {
    const int64_t T = (a.N / 128) * (a.Mp / 128);
    const int64_t W = a.part ? fp8_sk_shares(a.Mp, a.N, a.K) : 0, cus = cu_count();
    if (W) {  // the 8-wave shares of the W4A4 stream-K (the wide tile's shares measured slower: 100 -> 104 us)
        fp8_gemm_sk_kernel<256, 128, 64, 64, SK_NW, WDL_GEMM_STAGES><<<unsigned(W), SK_NW * 64, 0, stream>>>(a);
        const int rc = check_launch("fp8_gemm stream-K");
        if (rc) return rc;
        const unsigned tiles = unsigned((a.N / 256) * (a.Mp / 128));
        w4a4_merge_kernel<256, 128, 64, 64, SK_NW, EPI><<<tiles, SK_NW * 64, 0, stream>>>(a, W);
        return check_launch("fp8_gemm merge");
    }
    if (a.N % 256 == 0 && cus > 0 && 16 * (T / 2) >= 15 * cus) {
        fp8_gemm_kernel<256, 128, 128, 64, 4, EPI, 4><<<unsigned(T / 2), 256, 0, stream>>>(a);
        return check_launch("fp8_gemm");
    }
    fp8_gemm_kernel<128, 128, 64, 64, 4, EPI, 4><<<unsigned(T), 256, 0, stream>>>(a);
    return check_launch("fp8_gemm");
}

int launch_fp8(const GemmArgs& a, int epi, hipStream_t stream) {
    if (a.N % 128 || a.Mp % 128) return fail(WDL_EINVAL, "fp8_gemm: tile 128x128 does not divide N=%lld Mp=%lld",
                                             (long long)a.N, (long long)a.Mp);
    switch (epi) {
        case EPI_FP8_ROWS: return launch_fp8_epi<EPI_FP8_ROWS>(a, stream);
        case EPI_FP8_TENSOR: return launch_fp8_epi<EPI_FP8_TENSOR>(a, stream);
        default: return fail(WDL_EINVAL, "fp8_gemm: bad mode");
    }
}

// The fused GELU MLP's first GEMM always runs the one-pass 128 x 128 launch (its epilogue owns one 64-feature
// group per wave), then the low-rank partials of its N / 128 feature tiles are added per token.
int dispatch_gelu_quant(const GemmArgs& a, float* lora2, hipStream_t stream) {
    const unsigned grid = unsigned((a.N / 128) * (a.Mp / 128));
    w4a4_gemm_kernel<128, 128, 64, 64, 4, EPI_GELU_QUANT, WDL_GEMM_STAGES><<<grid, 256, 0, stream>>>(a);
    const int rc = check_launch("w4a4_gemm_gelu_quant");
    if (rc) return rc;
    return lora_sum(a.lpart, int(a.N / 128), a.Mp * 32, lora2, stream);
}

// fp6 codes (e3m2 of 2w) of the two's complement nibbles 0..7 (w = 0..7) and 8..15 (w = -8..-1)
constexpr uint32_t LUT0 = 0x16141000u, LUT1 = 0x1B1A1918u, LUT2 = 0x393A3B3Cu, LUT3 = 0x30343638u;

// four nibbles in the low 4 bits of each byte of x -> four 6-bit codes, one per byte
__device__ __forceinline__ uint32_t nib4_to_code6(uint32_t x) {
    const uint32_t sel = x & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(LUT1, LUT0, sel);
    const uint32_t neg = __builtin_amdgcn_perm(LUT3, LUT2, sel);
    const uint32_t t = (x >> 3) & 0x01010101u;
    const uint32_t mask = (t << 8) - t;  // 0xff in every byte whose nibble is negative
    return (neg & mask) | (pos & ~mask);
}

// weight scales -> the GEMM's pairs: hi = the scale truncated to bf16 (the scale itself when it is bf16), lo = the
// rest, exact in bf16 (an fp16 scale has 11 significant bits, hi takes 8), packed hi | lo << 16
__global__ __launch_bounds__(256) void scale_pairs_kernel(const uint16_t* s, int fp16, int64_t n, uint32_t* out) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= n) return;
    const uint16_t v = s[i];
    const float f = fp16 ? __half2float(__ushort_as_half(v)) : bf16_to_f32(v);
    const uint32_t fb = __float_as_uint(f);
    const float lo = f - __uint_as_float(fb & 0xffff0000u);  // exact
    out[i] = (fb >> 16) | (__float_as_uint(lo) & 0xffff0000u);
}

// packed nibbles [N, K/2] -> fp6 codes in the tile-blocked layout. The 32 packed bytes of a row's group hold
// value k = j in the low nibble and k = 32 + j in the high nibble of byte j, so the low nibbles are half 0 and the
// high nibbles half 1 (position j). One thread per 16 packed bytes: 16 codes of each half, 12 bytes each.
__global__ __launch_bounds__(256) void weight_codes_kernel(const uint4* qw, int64_t units, int64_t K, uint8_t* codes) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= units) return;
    const int64_t per_row = K / 32;  // 16-byte units per row
    const int64_t row = i / per_row, in_row = i % per_row;
    const int64_t g = in_row / 2;
    const int u = int(in_row % 2);   // positions 16u .. 16u + 15
    const uint4 w = qw[i];
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
    uint8_t* dst = codes + blocked6_offset(row, g, K);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        uint32_t q[4];  // 24-bit quads: positions 16u + 4j .. + 3
#pragma unroll
        for (int j = 0; j < 4; ++j) q[j] = pack4x6(nib4_to_code6((words[j] >> (4 * h)) & 0x0f0f0f0fu));
        const uint32_t d0 = q[0] | (q[1] << 24), d1 = (q[1] >> 8) | (q[2] << 16), d2 = (q[2] >> 16) | (q[3] << 8);
        // half bytes 12u .. 12u + 11
        *reinterpret_cast<uint32_t*>(dst + half_byte(h, 12 * u)) = d0;
        *reinterpret_cast<uint32_t*>(dst + half_byte(h, 12 * u + 4)) = d1;
        *reinterpret_cast<uint32_t*>(dst + half_byte(h, 12 * u + 8)) = d2;
    }
}

}  // namespace

// epilogue: 0 = bf16 out, 1 = fp32 out, 2 = out(bf16) = bf16(out + bf16(y) * gate) (gated residual in place),
// 3 = bf16(GELU_tanh(y)) out
extern "C" int64_t wdl_w4a4_gemm_workspace_bytes(int64_t Mp, int64_t N, int64_t K) {
    if (Mp <= 0 || Mp % 128 || N <= 0 || K <= 0 || K % 64) return 0;
    if (bal_fits(Mp, N, K)) return BAL_TOKEN_BYTES;
    return 2 * sk_shares(Mp, N, K) * SK_SLOT * int64_t(sizeof(float));
}

extern "C" int wdl_w4a4_gemm(const void* qa, const void* ascales, const void* wcodes, const void* wscales,
                             const float* lora, const void* proj_up, const void* bias, int64_t M, int64_t Mp,
                             int64_t N, int64_t K, int64_t rank, void* out, int64_t ldo, int epilogue,
                             const float* gate, float* ln_partials, void* workspace, hipStream_t stream) {
    if (M < 0 || Mp < M || Mp % 128 || N <= 0 || N % 128 || K <= 0 || K % 64 || K > (int64_t(1) << 30) || ldo < N ||
        ldo % 4)
        return fail(WDL_EINVAL, "w4a4_gemm: bad shape M=%lld Mp=%lld N=%lld K=%lld ldo=%lld", (long long)M,
                    (long long)Mp, (long long)N, (long long)K, (long long)ldo);
    if (lora && (rank != 32 || !proj_up)) return fail(WDL_EINVAL, "w4a4_gemm: low-rank branch needs rank 32");
    if (!qa || !ascales || !wcodes || !wscales || !out) return fail(WDL_EINVAL, "w4a4_gemm: null pointer");
    if ((reinterpret_cast<uintptr_t>(qa) | reinterpret_cast<uintptr_t>(wcodes)) % 16 ||
        (reinterpret_cast<uintptr_t>(ascales) | reinterpret_cast<uintptr_t>(wscales)) % 4)
        return fail(WDL_EINVAL, "w4a4_gemm: operands must be 16-byte (codes) / 4-byte (scales) aligned");
    if (epilogue == EPI_RESIDUAL && !gate) return fail(WDL_EINVAL, "w4a4_gemm: residual epilogue needs gate");
    if (reinterpret_cast<uintptr_t>(gate) % 16 || reinterpret_cast<uintptr_t>(bias) % 8 ||
        reinterpret_cast<uintptr_t>(out) % 16 || reinterpret_cast<uintptr_t>(proj_up) % 16 ||
        reinterpret_cast<uintptr_t>(lora) % 16 || (epilogue != EPI_F32 && ldo % 8))
        return fail(WDL_EINVAL, "w4a4_gemm: out, gate, lora and proj_up must be 16-byte aligned, bias 8-byte, and "
                                "bf16 output rows a multiple of 8 elements");
    if (ln_partials && (epilogue != EPI_RESIDUAL || reinterpret_cast<uintptr_t>(ln_partials) % 16))
        return fail(WDL_EINVAL, "w4a4_gemm: LayerNorm partials come with the residual epilogue, 16-byte aligned");
    if (M == 0) return WDL_OK;
    GemmArgs a{static_cast<const uint8_t*>(qa), static_cast<const uint16_t*>(ascales),
               static_cast<const uint8_t*>(wcodes), static_cast<const uint32_t*>(wscales), lora,
               static_cast<const uint16_t*>(proj_up), static_cast<const uint16_t*>(bias), M, Mp, N, K, out, ldo,
               gate, nullptr, nullptr, static_cast<float*>(workspace)};
    a.lnp = reinterpret_cast<float2*>(ln_partials);
    if (reinterpret_cast<uintptr_t>(workspace) % 16)
        return fail(WDL_EINVAL, "w4a4_gemm: workspace must be 16-byte aligned");
    return dispatch(a, epilogue, stream);
}

extern "C" int64_t wdl_w4a4_gemm_gelu_quant_workspace_floats(int64_t Mp, int64_t N) {
    if (Mp <= 0 || Mp % 128 || N <= 0 || N % 128) return 0;
    return (N / 128) * Mp * 32;
}

extern "C" int wdl_w4a4_gemm_gelu_quant(const void* qa, const void* ascales, const void* wcodes, const void* wscales,
                                        const float* lora, const void* proj_up, const void* bias, int64_t M,
                                        int64_t Mp, int64_t N, int64_t K, int64_t rank, const void* smooth2,
                                        const void* proj_down2_t, void* q2, void* ascales2, float* lora2,
                                        float* workspace, hipStream_t stream) {
    if (M < 0 || Mp < M || Mp % 128 || N <= 0 || N % 128 || K <= 0 || K % 64 || K > (int64_t(1) << 30))
        return fail(WDL_EINVAL, "w4a4_gemm_gelu_quant: bad shape M=%lld Mp=%lld N=%lld K=%lld", (long long)M,
                    (long long)Mp, (long long)N, (long long)K);
    if (lora && (rank != 32 || !proj_up)) return fail(WDL_EINVAL, "w4a4_gemm_gelu_quant: low-rank branch needs rank 32");
    if (!qa || !ascales || !wcodes || !wscales || !smooth2 || !proj_down2_t || !q2 || !ascales2 || !lora2 ||
        !workspace)
        return fail(WDL_EINVAL, "w4a4_gemm_gelu_quant: null pointer");
    const uintptr_t a16 = reinterpret_cast<uintptr_t>(qa) | reinterpret_cast<uintptr_t>(wcodes) |
                          reinterpret_cast<uintptr_t>(q2) | reinterpret_cast<uintptr_t>(lora2) |
                          reinterpret_cast<uintptr_t>(workspace) | reinterpret_cast<uintptr_t>(proj_up) |
                          reinterpret_cast<uintptr_t>(lora);
    const uintptr_t a8 = reinterpret_cast<uintptr_t>(bias) | reinterpret_cast<uintptr_t>(smooth2) |
                         reinterpret_cast<uintptr_t>(proj_down2_t);
    if (a16 % 16 || a8 % 8 || (reinterpret_cast<uintptr_t>(ascales) | reinterpret_cast<uintptr_t>(wscales) |
                               reinterpret_cast<uintptr_t>(ascales2)) % 4)
        return fail(WDL_EINVAL, "w4a4_gemm_gelu_quant: codes, lora, proj_up and workspace must be 16-byte aligned, "
                                "bias, smooth2 and proj_down2_t 8-byte, scales 4-byte");
    if (M == 0) return WDL_OK;
    GemmArgs a{static_cast<const uint8_t*>(qa), static_cast<const uint16_t*>(ascales),
               static_cast<const uint8_t*>(wcodes), static_cast<const uint32_t*>(wscales), lora,
               static_cast<const uint16_t*>(proj_up), static_cast<const uint16_t*>(bias), M, Mp, N, K, nullptr, N,
               nullptr, nullptr, nullptr, nullptr, static_cast<uint8_t*>(q2), static_cast<uint16_t*>(ascales2),
               static_cast<const uint16_t*>(smooth2), static_cast<const uint16_t*>(proj_down2_t), workspace};
    return dispatch_gelu_quant(a, lora2, stream);
}

extern "C" int wdl_w4a4_scale_pairs(const void* scales, int fp16, int64_t n, void* pairs, hipStream_t stream) {
    if (n < 0) return fail(WDL_EINVAL, "w4a4_scale_pairs: bad count %lld", (long long)n);
    if (n == 0) return WDL_OK;
    if (!scales || !pairs) return fail(WDL_EINVAL, "w4a4_scale_pairs: null pointer");
    if (reinterpret_cast<uintptr_t>(scales) % 2 || reinterpret_cast<uintptr_t>(pairs) % 4)
        return fail(WDL_EINVAL, "w4a4_scale_pairs: scales must be 2-byte and pairs 4-byte aligned");
    scale_pairs_kernel<<<unsigned((n + 255) / 256), 256, 0, stream>>>(static_cast<const uint16_t*>(scales), fp16 != 0,
                                                                     n, static_cast<uint32_t*>(pairs));
    return check_launch("w4a4_scale_pairs");
}

extern "C" int wdl_w4a4_weight_codes(const void* qweight, int64_t N, int64_t K, void* codes, hipStream_t stream) {
    if (N < 0 || N % BLOCK_ROWS || K <= 0 || K % 64)
        return fail(WDL_EINVAL, "w4a4_weight_codes: bad shape N=%lld K=%lld (N %% 128 == 0, K %% 64 == 0)",
                    (long long)N, (long long)K);
    if (!qweight || !codes) return fail(WDL_EINVAL, "w4a4_weight_codes: null pointer");
    if ((reinterpret_cast<uintptr_t>(qweight) | reinterpret_cast<uintptr_t>(codes)) % 16)
        return fail(WDL_EINVAL, "w4a4_weight_codes: buffers must be 16-byte aligned");
    const int64_t units = N * K / 32;
    if (units == 0) return WDL_OK;
    weight_codes_kernel<<<unsigned((units + 255) / 256), 256, 0, stream>>>(static_cast<const uint4*>(qweight), units,
                                                                          K, static_cast<uint8_t*>(codes));
    return check_launch("w4a4_weight_codes");
}

extern "C" int64_t wdl_fp8_gemm_workspace_bytes(int64_t Mp, int64_t N, int64_t K) {
    if (Mp <= 0 || Mp % 128 || N <= 0 || K <= 0 || K % 64) return 0;
    return 2 * fp8_sk_shares(Mp, N, K) * SK_SLOT * int64_t(sizeof(float));
}

extern "C" int wdl_fp8_gemm(const void* xq, const float* x_scale, const void* wq, const float* w_scale,
                            const void* bias, int64_t M, int64_t Mp, int64_t N, int64_t K, int rows, void* out,
                            int64_t ldo, void* workspace, hipStream_t stream) {
    if (M < 0 || Mp < M || Mp % 128 || N <= 0 || N % 128 || K <= 0 || K % 64 || K > (int64_t(1) << 30) || ldo < N ||
        ldo % 4)
        return fail(WDL_EINVAL, "fp8_gemm: bad shape M=%lld Mp=%lld N=%lld K=%lld ldo=%lld", (long long)M,
                    (long long)Mp, (long long)N, (long long)K, (long long)ldo);
    if (!xq || !x_scale || !wq || !w_scale || !out) return fail(WDL_EINVAL, "fp8_gemm: null pointer");
    if ((reinterpret_cast<uintptr_t>(xq) | reinterpret_cast<uintptr_t>(wq)) % 16)
        return fail(WDL_EINVAL, "fp8_gemm: operands must be 16-byte aligned");
    if (reinterpret_cast<uintptr_t>(bias) % 8 || reinterpret_cast<uintptr_t>(out) % 8 ||
        (rows && reinterpret_cast<uintptr_t>(w_scale) % 16))
        return fail(WDL_EINVAL, "fp8_gemm: bias and out must be 8-byte aligned, row scales 16-byte");
    if (M == 0) return WDL_OK;
    if (reinterpret_cast<uintptr_t>(workspace) % 16) return fail(WDL_EINVAL, "fp8_gemm: workspace must be 16-byte aligned");
    // the stream-K launch runs only with a workspace of the queried size; any other shape ignores it
    float* part = workspace && wdl_fp8_gemm_workspace_bytes(Mp, N, K) ? static_cast<float*>(workspace) : nullptr;
    GemmArgs a{static_cast<const uint8_t*>(xq), nullptr, static_cast<const uint8_t*>(wq), nullptr, nullptr, nullptr,
               static_cast<const uint16_t*>(bias), M, Mp, N, K, out, ldo, nullptr, x_scale, w_scale, part};
    return launch_fp8(a, rows ? EPI_FP8_ROWS : EPI_FP8_TENSOR, stream);
}
