// FP8 weight-only linear on gfx950: y = x W^T (W = w_fp8 * w_scale) + bias, x and y bf16. The weight stays in e4m3
// in memory (one byte per value, per output row or per tensor scale); activations keep their bf16 precision. No
// counterpart in the reference, whose FP8 linears quantize the activation too (quantization/fp8.py:1-6, 44-67): the
// mixed-precision mode of the benchmark plan (attention projections FP8 weight-only, FFN W4A4).
//
// Products. Every e4m3 value is exact in bf16 (3 mantissa bits, exponents inside bf16's range), so the weight codes
// are widened to bf16 in registers and C^T = W X^T runs on v_mfma_f32_32x32x16_bf16: each product of a bf16 and an
// e4m3 value is exact in fp32 (8 + 4 significant bits), sums accumulate in fp32, and the per-row scale multiplies
// the sum once in the epilogue (scale * sum, then + bias, then bf16).
//
// Tiles. A workgroup of 4 waves computes a 128 (features) x 128 (tokens) tile, each wave 32 features x 128 tokens
// (4 subtiles of 32 x 32), so a lane owns one token and 16 features per subtile, and every weight row of the tile is
// widened by one wave only, once per 16-deep step for four MFMAs (64 x 64 wave tiles widened each row twice, for two
// MFMAs: 7-11 % slower). K advances 64 per stage through a 3-stage LDS ring
// fed by direct global->LDS loads (16 bytes per lane, 6 per wave per stage, waited for with an explicit vmcnt):
//   W stage: [128 rows][64 B] of e4m3, each row's four 16-byte quarters XOR-swizzled by (row / 4) % 4;
//   X stage: [128 rows][128 B] of bf16, each row's eight 16-byte chunks XOR-swizzled by row % 8,
// so the 8- and 16-byte fragment reads of 32 consecutive rows spread over the banks. Rows of X past M are loaded
// from row M - 1 (never written back). 72 KB of LDS and two workgroups per CU; tile ids are remapped so that the
// tiles of one weight slab run on one XCD.
#include "wdl_common.h"

namespace {

using namespace wdl;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int BN = 128, BM = 128, KS = 64, STAGES = 3;
constexpr int WST = BN * KS;          // bytes of a W stage (e4m3)
constexpr int XST = BM * KS * 2;      // bytes of an X stage (bf16)
constexpr int LPG = (WST + XST) / (256 * 16);  // 16-byte loads per lane per stage: 6
constexpr int EPI_BF16 = 0, EPI_RESIDUAL = 2;

struct Args {
    const uint16_t* x;
    int64_t ldx;
    const uint8_t* w;
    const float* ws;      // [N] (rows) or [1]
    int64_t ws_step;      // 1 (rows) or 0 (tensor)
    const uint16_t* bias; // [N] or null
    uint16_t* out;
    int64_t ldo;
    const float* gate;    // [N] (gated residual)
    int64_t M, N, K, ntm;
};

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// 64 lanes x 16 bytes from a wave-uniform base plus a 32-bit per-lane offset to LDS [m0, m0 + 1024)
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// eight e4m3 codes (little-endian in two dwords) -> eight bf16 (exact: the e4m3 value's fp32 form truncated)
__device__ __forceinline__ bf16x8 widen(uint2 c) {
    const auto f0 = __builtin_amdgcn_cvt_pk_f32_fp8(int(c.x), false), f1 = __builtin_amdgcn_cvt_pk_f32_fp8(int(c.x), true);
    const auto f2 = __builtin_amdgcn_cvt_pk_f32_fp8(int(c.y), false), f3 = __builtin_amdgcn_cvt_pk_f32_fp8(int(c.y), true);
    auto pack = [](float lo, float hi) { return (__float_as_uint(lo) >> 16) | (__float_as_uint(hi) & 0xffff0000u); };
    return __builtin_bit_cast(bf16x8, make_uint4(pack(f0[0], f0[1]), pack(f1[0], f1[1]), pack(f2[0], f2[1]),
                                                 pack(f3[0], f3[1])));
}

template <int EPI>
__global__ __launch_bounds__(256) void fp8wo_gemm_kernel(Args a) {
    __shared__ __attribute__((aligned(1024))) uint8_t sW[STAGES][WST];
    __shared__ __attribute__((aligned(1024))) uint8_t sX[STAGES][XST];

    const int t = threadIdx.x, lane = t % 64, half = lane / 32, tok = lane % 32;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);
    const int wn = wave;  // the wave's 32 feature rows of the tile, against all 128 tokens
    const int64_t total = gridDim.x, pid = blockIdx.x;
    const int64_t tile = total % 8 == 0 ? (pid % 8) * (total / 8) + pid / 8 : pid;
    const int64_t n0 = (tile / a.ntm) * BN, m0 = (tile % a.ntm) * BM;

    // this lane's load offsets: W chunk id = 64 (4 i + wave) + lane (i < 2): row id / 4, stored quarter id % 4 holds
    // the row's quarter (id % 4) ^ ((row / 4) % 4); X chunk id (i < 4): row id / 8, stored chunk id % 8 holds chunk
    // (id % 8) ^ (row % 8)
    uint32_t woff[2], xoff[4];
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        const int id = 64 * (4 * i + wave) + lane, row = id / 4, q = (id % 4) ^ ((row / 4) % 4);
        woff[i] = uint32_t(row * a.K + 16 * q);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int id = 64 * (4 * i + wave) + lane, row = id / 8, c = (id % 8) ^ (row % 8);
        const int64_t m = m0 + row < a.M ? m0 + row : a.M - 1;
        xoff[i] = uint32_t(m * a.ldx * 2 + 16 * c);
    }
    const uint8_t* wtile = a.w + n0 * a.K;
    const int G = int(a.K / KS);
    auto issue = [&](int slot, int g) {
        const int gg = g < G ? g : G - 1;  // past the end: the last stage again (a slot no wave reads any more)
        const uint8_t* wb = wtile + int64_t(gg) * KS;
        const uint8_t* xb = reinterpret_cast<const uint8_t*>(a.x) + int64_t(gg) * KS * 2;
#pragma unroll
        for (int i = 0; i < 2; ++i) dma16s(wb, woff[i], lds_addr(&sW[slot][1024 * (4 * i + wave)]));
#pragma unroll
        for (int i = 0; i < 4; ++i) dma16s(xb, xoff[i], lds_addr(&sX[slot][1024 * (4 * i + wave)]));
    };

    f32x16 acc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[j] = f32x16{};

    // fragment rows of this lane: W row 32 wn + tok, X rows 32 j + tok
    const int wsw = ((tok / 4) % 4), xsw = tok % 8;  // (32 wn and 32 j leave both unchanged)
    issue(0, 0);
    issue(1, 1);
    for (int g = 0; g < G; ++g) {
        wait_vmcnt<LPG>();  // stage g landed (g + 1 may be in flight)
        __syncthreads();
        issue((g + 2) % STAGES, g + 2);
        const uint8_t* W = sW[g % STAGES];
        const uint8_t* X = sX[g % STAGES];
#pragma unroll
        for (int s = 0; s < 4; ++s) {  // 16-deep steps: quarter s of the rows, k = 16 s + 8 half .. + 7
            bf16x8 bf[4];
            const bf16x8 af = widen(*reinterpret_cast<const uint2*>(W + (32 * wn + tok) * 64 + 16 * (s ^ wsw) + 8 * half));
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint8_t* row = X + (32 * j + tok) * 128;
                bf[j] = *reinterpret_cast<const bf16x8*>(row + 16 * ((2 * s + half) ^ xsw));
            }
#pragma unroll
            for (int j = 0; j < 4; ++j) acc[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, bf[j], acc[j], 0, 0, 0);
        }
    }
    wait_vmcnt<0>();  // the clamped tail loads land before the workgroup ends

    // epilogue: element e of subtile j is feature n0 + 32 wn + 8 (e / 4) + 4 half + e % 4 of token m0 + 32 j + tok;
    // four consecutive features per 8-byte store
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int64_t m = m0 + 32 * j + tok;
        if (m >= a.M) continue;
        uint16_t* orow = a.out + m * a.ldo;
#pragma unroll
        for (int i = 0; i < 1; ++i)
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int64_t n = n0 + 32 * wn + 8 * q + 4 * half;
                uint16_t r[4];
                uint2 old = make_uint2(0u, 0u);
                if (EPI == EPI_RESIDUAL) old = *reinterpret_cast<const uint2*>(orow + n);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    float y = acc[j][4 * q + e] * a.ws[(n + e) * a.ws_step];
                    if (a.bias) y = y + bf16_to_f32(a.bias[n + e]);
                    if (EPI == EPI_RESIDUAL) {
                        const uint16_t o = uint16_t(((e < 2 ? old.x : old.y) >> (16 * (e % 2))) & 0xffffu);
                        y = bf16_to_f32(o) + bf16_to_f32(f32_to_bf16(y)) * a.gate[n + e];
                    }
                    r[e] = f32_to_bf16(y);
                }
                *reinterpret_cast<uint2*>(orow + n) = make_uint2(r[0] | (uint32_t(r[1]) << 16),
                                                                 r[2] | (uint32_t(r[3]) << 16));
            }
    }
}

}  // namespace

extern "C" int wdl_fp8wo_gemm(const void* x, int64_t ldx, const void* w, const float* w_scale, int scale_rows,
                              const void* bias, int64_t M, int64_t N, int64_t K, void* out, int64_t ldo,
                              int epilogue, const float* gate, hipStream_t stream) {
    if (M < 0 || N <= 0 || K <= 0 || N % BN || K % KS || ldx < K || ldo < N || ldx % 8 || ldo % 4)
        return fail(WDL_EINVAL, "fp8wo_gemm: bad shape M=%lld N=%lld K=%lld ldx=%lld ldo=%lld", (long long)M,
                    (long long)N, (long long)K, (long long)ldx, (long long)ldo);
    if (!x || !w || !w_scale || !out || (epilogue == EPI_RESIDUAL && !gate))
        return fail(WDL_EINVAL, "fp8wo_gemm: null pointer");
    if (epilogue != EPI_BF16 && epilogue != EPI_RESIDUAL)
        return fail(WDL_EINVAL, "fp8wo_gemm: epilogue must be 0 (bf16) or 2 (gated residual)");
    if ((reinterpret_cast<uintptr_t>(x) | reinterpret_cast<uintptr_t>(w)) % 16 ||
        reinterpret_cast<uintptr_t>(out) % 8 || reinterpret_cast<uintptr_t>(bias) % 2)
        return fail(WDL_EINVAL, "fp8wo_gemm: x, w 16-byte aligned, out 8-byte, bias 2-byte");
    if (int64_t(BN) * K >= (int64_t(1) << 31) || M * ldx * 2 >= (int64_t(1) << 32))
        return fail(WDL_EINVAL, "fp8wo_gemm: operands beyond 32-bit load offsets");
    if (M == 0) return WDL_OK;
    const int64_t ntm = (M + BM - 1) / BM, tiles = ntm * (N / BN);
    Args a{static_cast<const uint16_t*>(x), ldx, static_cast<const uint8_t*>(w), w_scale, scale_rows ? 1 : 0,
           static_cast<const uint16_t*>(bias), static_cast<uint16_t*>(out), ldo, gate, M, N, K, ntm};
    if (epilogue == EPI_RESIDUAL) fp8wo_gemm_kernel<EPI_RESIDUAL><<<unsigned(tiles), 256, 0, stream>>>(a);
    else fp8wo_gemm_kernel<EPI_BF16><<<unsigned(tiles), 256, 0, stream>>>(a);
    return check_launch("fp8wo_gemm");
}
