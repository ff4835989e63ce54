// W4A4 GEMM of the SVDQuant linears on gfx950 matrix cores.
//
//   y[m][n] = sum_g as[g][m] * ws[g][n] * I_g[m][n]  +  bf16(lora[m]) . pu[n]  +  bias[n]
//   I_g[m][n] = sum_{k in group g} qa[m][k] * qw[n][k]          (exact integers)
//
// Operands: qa — activation int4 values as e4m3 codes, one byte each, [Mp, K] (wdl_act_quant_w4);
// qw — weight int4 nibbles [N, K/2], in each 64-group byte j holds k = j (low nibble) and k = j + 32 (high),
// two's complement; as [K/64, Mp], ws [K/64, N] bf16; lora fp32 [Mp, 32]; pu bf16 [N, 32]; bias bf16 [N].
//
// Arithmetic: every int4 value is exactly an e4m3 value, so v_mfma_f32_32x32x64_f8f6f4 (one 64-deep group per
// instruction, the int8 rate) returns I_g exactly as an fp32 integer (|I_g| <= 64 * 8 * 15 < 2^24). The per-group
// scale product ws[n] * as[m] comes from a bf16 outer-product MFMA (exact: 8-bit by 8-bit significands), and each
// group is folded in with one fmaf per element, groups in increasing order. The low-rank term is two bf16 MFMAs
// accumulated into the result, then the bias.
//
// Orientation: the tile is computed transposed, C^T[n][m] (rows = output features, columns = tokens), so a lane
// holds one token and 16 features: row n = 8*(i/4) + 4*(lane/32) + i%4, column m = lane%32 of each 32x32 subtile.
// Weights are unpacked once per workgroup per group into LDS as e4m3 codes (two v_perm lookups per 4 values).
#include "wdl_common.h"

namespace {

using namespace wdl;

typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

enum Epilogue { EPI_BF16 = 0, EPI_F32 = 1, EPI_RESIDUAL = 2, EPI_GELU = 3 };

// GELU, tanh form: 0.5 x (1 + tanh(sqrt(2/pi) (x + 0.044715 x^3))), tanh(u) = 1 - 2 / (exp(2u) + 1)
__device__ __forceinline__ float gelu_tanh(float x) {
    const float u = 0.7978845608028654f * (x + 0.044715f * x * x * x);
    const float th = 1.0f - 2.0f / (__expf(2.0f * u) + 1.0f);
    return 0.5f * x * (1.0f + th);
}

struct GemmArgs {
    const uint8_t* qa;        // [Mp, K] e4m3 codes
    const uint16_t* as;       // [G, Mp]
    const uint8_t* qw;        // [N, K/2]
    const uint16_t* ws;       // [G, N]
    const float* lora;        // [Mp, 32] or null
    const uint16_t* pu;       // [N, 32] or null
    const uint16_t* bias;     // [N] or null
    int64_t M, Mp, N, K;
    void* out;                // bf16 / fp32 [M, ldo]
    int64_t ldo;
    const float* gate;        // [N] fp32 (EPI_RESIDUAL: out += gate * bf16(y))
};

constexpr int PADK = 80;  // LDS row stride (bytes) of 64-byte k rows

// e4m3 codes of the two's complement nibbles 0..7 (values 0..7) and 8..15 (values -8..-1)
constexpr uint32_t LUT0 = 0x44403800u, LUT1 = 0x4E4C4A48u, LUT2 = 0xCACCCED0u, LUT3 = 0xB8C0C4C8u;

// four nibbles in the low 4 bits of each byte of x -> four e4m3 codes
__device__ __forceinline__ uint32_t nib4_to_e4m3(uint32_t x) {
    const uint32_t sel = x & 0x07070707u;
    const uint32_t pos = __builtin_amdgcn_perm(LUT1, LUT0, sel);
    const uint32_t neg = __builtin_amdgcn_perm(LUT3, LUT2, sel);
    const uint32_t t = (x >> 3) & 0x01010101u;
    const uint32_t mask = (t << 8) - t;  // 0xff in every byte whose nibble is negative
    return (neg & mask) | (pos & ~mask);
}

template <int BN, int BM, int WN, int WM, int EPI>
__global__ __launch_bounds__(256) void w4a4_gemm_kernel(GemmArgs p) {
    static_assert((BN / WN) * (BM / WM) == 4, "4 waves");
    constexpr int TN = WN / 32, TM = WM / 32;
    __shared__ __attribute__((aligned(16))) uint8_t sW[2][BN * PADK];
    __shared__ __attribute__((aligned(16))) uint8_t sX[2][BM * PADK];
    __shared__ uint16_t sWs[2][BN];
    __shared__ uint16_t sAs[2][BM];

    const int t = threadIdx.x, lane = t % 64, wave = t / 64;
    const int wn = wave % (BN / WN), wm = wave / (BN / WN);
    const int64_t n0 = int64_t(blockIdx.x) * BN, m0 = int64_t(blockIdx.y) * BM;
    const int64_t K = p.K, G = K / 64;

    // global -> register staging of one group
    constexpr int WCH = BN * 2 / 256;  // 16-byte chunks of packed weights per thread
    constexpr int XCH = BM * 4 / 256;  // 16-byte chunks of activation codes per thread
    static_assert(WCH >= 1 && XCH >= 1, "tile too small for 256 threads");
    uint4 wreg[WCH], xreg[XCH];
    uint16_t wsreg = 0, asreg = 0;

    auto fetch = [&](int64_t g) {
#pragma unroll
        for (int c = 0; c < WCH; ++c) {
            const int chunk = t + 256 * c, row = chunk / 2, half = chunk % 2;
            wreg[c] = *reinterpret_cast<const uint4*>(p.qw + (n0 + row) * (K / 2) + g * 32 + half * 16);
        }
#pragma unroll
        for (int c = 0; c < XCH; ++c) {
            const int chunk = t + 256 * c, row = chunk / 4, quarter = chunk % 4;
            xreg[c] = *reinterpret_cast<const uint4*>(p.qa + (m0 + row) * K + g * 64 + quarter * 16);
        }
        if (t < BN) wsreg = p.ws[g * p.N + n0 + t];
        if (t < BM) asreg = p.as[g * p.Mp + m0 + t];
    };
    auto stash = [&](int st) {
#pragma unroll
        for (int c = 0; c < WCH; ++c) {
            const int chunk = t + 256 * c, row = chunk / 2, half = chunk % 2;
            const uint32_t w[4] = {wreg[c].x, wreg[c].y, wreg[c].z, wreg[c].w};
            uint32_t lo[4], hi[4];
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                lo[j] = nib4_to_e4m3(w[j] & 0x0f0f0f0fu);
                hi[j] = nib4_to_e4m3((w[j] >> 4) & 0x0f0f0f0fu);
            }
            uint8_t* dst = &sW[st][row * PADK];
            *reinterpret_cast<uint4*>(dst + half * 16) = make_uint4(lo[0], lo[1], lo[2], lo[3]);
            *reinterpret_cast<uint4*>(dst + 32 + half * 16) = make_uint4(hi[0], hi[1], hi[2], hi[3]);
        }
#pragma unroll
        for (int c = 0; c < XCH; ++c) {
            const int chunk = t + 256 * c, row = chunk / 4, quarter = chunk % 4;
            *reinterpret_cast<uint4*>(&sX[st][row * PADK + quarter * 16]) = xreg[c];
        }
        if (t < BN) sWs[st][t] = wsreg;
        if (t < BM) sAs[st][t] = asreg;
    };

    f32x16 acc[TN][TM];
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) acc[i][j] = f32x16{};
    const f32x16 zero = {};

    fetch(0);
    stash(0);
    for (int64_t g = 0; g < G; ++g) {
        const int st = int(g & 1);
        __syncthreads();
        if (g + 1 < G) fetch(g + 1);
        i32x8 af[TN], bf[TM];
        i16x4 sa[TN], sb[TM];
#pragma unroll
        for (int i = 0; i < TN; ++i) {
            const int row = wn * WN + i * 32 + lane % 32;
            const uint8_t* src = &sW[st][row * PADK + 32 * (lane / 32)];
            const uint4 a0 = *reinterpret_cast<const uint4*>(src), a1 = *reinterpret_cast<const uint4*>(src + 16);
            af[i] = i32x8{int(a0.x), int(a0.y), int(a0.z), int(a0.w), int(a1.x), int(a1.y), int(a1.z), int(a1.w)};
            sa[i] = i16x4{short(lane < 32 ? sWs[st][row] : 0), 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const int row = wm * WM + j * 32 + lane % 32;
            const uint8_t* src = &sX[st][row * PADK + 32 * (lane / 32)];
            const uint4 b0 = *reinterpret_cast<const uint4*>(src), b1 = *reinterpret_cast<const uint4*>(src + 16);
            bf[j] = i32x8{int(b0.x), int(b0.y), int(b0.z), int(b0.w), int(b1.x), int(b1.y), int(b1.z), int(b1.w)};
            sb[j] = i16x4{short(lane < 32 ? sAs[st][row] : 0), 0, 0, 0};
        }
#pragma unroll
        for (int i = 0; i < TN; ++i)
#pragma unroll
            for (int j = 0; j < TM; ++j) {
                const f32x16 I = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[i], bf[j], zero, 0, 0, 0, 0, 0, 0);
                const f32x16 P = __builtin_amdgcn_mfma_f32_32x32x8bf16_1k(sa[i], sb[j], zero, 0, 0, 0);
#pragma unroll
                for (int e = 0; e < 16; ++e) acc[i][j][e] = fmaf(I[e], P[e], acc[i][j][e]);
            }
        if (g + 1 < G) stash(st ^ 1);
    }

    // low-rank branch: acc += pu[n] . bf16(lora[m]) over r = 0..31, two 32x32x16 bf16 MFMAs per subtile
    if (p.lora) {
#pragma unroll
        for (int i = 0; i < TN; ++i) {
            const int64_t n = n0 + wn * WN + i * 32 + lane % 32;
#pragma unroll
            for (int h = 0; h < 2; ++h) {
                const bf16x8 pa = *reinterpret_cast<const bf16x8*>(p.pu + n * 32 + h * 16 + 8 * (lane / 32));
#pragma unroll
                for (int j = 0; j < TM; ++j) {
                    const int64_t m = m0 + wm * WM + j * 32 + lane % 32;
                    const float* lr = p.lora + m * 32 + h * 16 + 8 * (lane / 32);
                    bf16x8 lb;
#pragma unroll
                    for (int e = 0; e < 8; ++e) lb[e] = __builtin_bit_cast(__bf16, f32_to_bf16(lr[e]));
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(pa, lb, acc[i][j], 0, 0, 0);
                }
            }
        }
    }

    // epilogue
#pragma unroll
    for (int i = 0; i < TN; ++i)
#pragma unroll
        for (int j = 0; j < TM; ++j) {
            const int64_t m = m0 + wm * WM + j * 32 + lane % 32;
            if (m >= p.M) continue;
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t nb = n0 + wn * WN + i * 32 + 8 * q + 4 * (lane / 32);
                float y[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    y[e] = acc[i][j][4 * q + e];
                    if (p.bias) y[e] = y[e] + bf16_to_f32(p.bias[nb + e]);
                }
                if (EPI == EPI_F32) {
                    float* o = static_cast<float*>(p.out) + m * p.ldo + nb;
                    *reinterpret_cast<float4*>(o) = make_float4(y[0], y[1], y[2], y[3]);
                } else {
                    uint16_t* o = static_cast<uint16_t*>(p.out) + m * p.ldo + nb;
                    uint16_t r[4];
                    if (EPI == EPI_RESIDUAL) {
                        const uint2 old = *reinterpret_cast<const uint2*>(o);
                        const uint16_t ov[4] = {uint16_t(old.x), uint16_t(old.x >> 16), uint16_t(old.y),
                                                uint16_t(old.y >> 16)};
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            const float yb = bf16_to_f32(f32_to_bf16(y[e]));
                            r[e] = f32_to_bf16(bf16_to_f32(ov[e]) + yb * p.gate[nb + e]);
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
}

template <int BN, int BM, int WN, int WM>
int launch(const GemmArgs& a, int epi, hipStream_t stream) {
    dim3 grid(unsigned(a.N / BN), unsigned(a.Mp / BM));
    switch (epi) {
        case EPI_BF16: w4a4_gemm_kernel<BN, BM, WN, WM, EPI_BF16><<<grid, 256, 0, stream>>>(a); break;
        case EPI_F32: w4a4_gemm_kernel<BN, BM, WN, WM, EPI_F32><<<grid, 256, 0, stream>>>(a); break;
        case EPI_RESIDUAL: w4a4_gemm_kernel<BN, BM, WN, WM, EPI_RESIDUAL><<<grid, 256, 0, stream>>>(a); break;
        case EPI_GELU: w4a4_gemm_kernel<BN, BM, WN, WM, EPI_GELU><<<grid, 256, 0, stream>>>(a); break;
        default: return fail(WDL_EINVAL, "w4a4_gemm: bad epilogue %d", epi);
    }
    return check_launch("w4a4_gemm");
}

}  // namespace

// epilogue: 0 = bf16 out, 1 = fp32 out, 2 = out(bf16) = bf16(out + bf16(y) * gate) (gated residual in place),
// 3 = bf16(GELU_tanh(y)) out
extern "C" int wdl_w4a4_gemm(const void* qa, const void* ascales, const void* qweight, const void* wscales,
                             const float* lora, const void* proj_up, const void* bias, int64_t M, int64_t Mp,
                             int64_t N, int64_t K, int64_t rank, void* out, int64_t ldo, int epilogue,
                             const float* gate, hipStream_t stream) {
    if (M < 0 || Mp < M || Mp % 128 || N <= 0 || N % 128 || K <= 0 || K % 64 || ldo < N || ldo % 4)
        return fail(WDL_EINVAL, "w4a4_gemm: bad shape M=%lld Mp=%lld N=%lld K=%lld ldo=%lld", (long long)M,
                    (long long)Mp, (long long)N, (long long)K, (long long)ldo);
    if (lora && (rank != 32 || !proj_up)) return fail(WDL_EINVAL, "w4a4_gemm: low-rank branch needs rank 32");
    if (!qa || !ascales || !qweight || !wscales || !out) return fail(WDL_EINVAL, "w4a4_gemm: null pointer");
    if (epilogue == EPI_RESIDUAL && !gate) return fail(WDL_EINVAL, "w4a4_gemm: residual epilogue needs gate");
    if (Mp == 0) return WDL_OK;
    GemmArgs a{static_cast<const uint8_t*>(qa), static_cast<const uint16_t*>(ascales),
               static_cast<const uint8_t*>(qweight), static_cast<const uint16_t*>(wscales), lora,
               static_cast<const uint16_t*>(proj_up), static_cast<const uint16_t*>(bias), M, Mp, N, K, out, ldo,
               gate};
    return launch<128, 128, 64, 64>(a, epilogue, stream);
}
