// Per-token, per-64-channel activation quantizer of the W4A4 linears, optionally fused with the LayerNorm and the
// adaLN modulation that precede it, and with the down projection of the low-rank branch.
//
// For rows m < M of x (bf16 [M, K], row stride ldx):
//   v     = x                                                       (plain), or
//   v     = bf16( LN(x)[*w + b] * (1 + mod_scale) + mod_shift )    (fused; fp32 math, one rounding)
//   u     = (v + qshift) / smooth                                   (IEEE fp32)
//   scale = bf16( max_{64 group} |u| / qmax )                       (qmax 7 signed, 15 unsigned)
//   q     = clamp(rint(u / scale))                                  (0 where scale is 0)
//   lora  = v . proj_down                                           (bf16 MFMA, fp32 sums)
// Outputs: q as e4m3 codes of the integer values (exact), one byte per value [Mp, K] (rows >= M zero);
// ascales bf16 [K/64, Mp]; lora fp32 [Mp, 32].
//
// Launches (all parallel over rows and column blocks, nothing serial over K):
//   row_stats  (LN only): one wave per row; LN statistics in a fixed order — lane l owns the 8-value chunks
//              c = l, l + 64, ... and sums them value by value; the 64 lane sums meet in an xor butterfly
//              (32, 16, 8, 4, 2, 1); mean = sum / K, var = sum((x - mean)^2) / K, rstd = 1 / sqrt(var + eps).
//   quant      grid (Mp / 32, ceil(K / 512)): 32 rows x 512 columns per workgroup, thread t owns row t / 8 and the
//              8 columns (t % 8) * 8 .. of each 64-group; the low-rank product over those 512 columns is a
//              32 x 32 partial (bf16 MFMA, the 4 waves' k-quarters summed in order).
//   lora_sum   lora = sum of the column-block partials in increasing order (only when K > 512).
#include "wdl_common.h"

namespace {

using namespace wdl;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int ROWS = 32;
constexpr int RANK = 32;
constexpr int CB = 512;  // columns per workgroup of the quant launch
constexpr int MAXCH = 8; // row_stats keeps up to 8 chunks per lane in registers (K <= 4096)

__device__ __forceinline__ void load8(const uint16_t* p, float* f) {
    uint4 raw = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = __uint_as_float(w[j] << 16);
        f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
}

__device__ __forceinline__ float butterfly64(float s) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) s = s + __shfl_xor(s, o);
    return s;
}

__global__ __launch_bounds__(256) void row_stats_kernel(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                                                        float eps, float2* stats) {
    const int lane = threadIdx.x % 64;
    const int64_t row = int64_t(blockIdx.x) * 4 + threadIdx.x / 64;
    if (row >= M) return;
    const uint16_t* xr = x + row * ldx;
    const int64_t chunks = K / 8;
    float v[MAXCH][8];
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
        const int64_t c = lane + 64 * i;
        if (c < chunks) load8(xr + c * 8, v[i]);
        else
            for (int j = 0; j < 8; ++j) v[i][j] = 0.0f;
    }
    float s = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXCH; ++i)
#pragma unroll
        for (int j = 0; j < 8; ++j) s = s + v[i][j];
    const float mean = butterfly64(s) / float(K);
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < MAXCH; ++i) {
        const bool real = lane + 64 * i < chunks;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float d = v[i][j] - mean;
            ss = ss + (real ? d * d : 0.0f);
        }
    }
    const float var = butterfly64(ss) / float(K);
    if (lane == 0) stats[row] = make_float2(mean, 1.0f / sqrtf(var + eps));
}

struct QuantArgs {
    const uint16_t* x;
    int64_t ldx;
    int64_t M, Mp, K;
    const uint16_t* smooth;    // bf16 [K]
    float qshift;
    int unsigned_q;
    const uint16_t* pdt;       // bf16 [RANK, K] (proj_down transposed), or null (no low-rank branch)
    uint8_t* q;                // [Mp, K]
    uint16_t* ascales;         // [K/64, Mp]
    float* lora;               // [nblocks, Mp, RANK] partials (or [Mp, RANK] when nblocks == 1)
    const float2* stats;       // LN (mean, rstd) per row, or null (no LN)
    const float* mod_shift;    // fp32 [K] or null
    const float* mod_scale;    // fp32 [K] or null (used as 1 + scale)
    const float* ln_w;         // fp32 [K] or null
    const float* ln_b;         // fp32 [K] or null
    uint16_t* v_out;           // bf16 [M, K] copy of v, or null
};

__global__ __launch_bounds__(256) void quant_kernel(QuantArgs a) {
    __shared__ __attribute__((aligned(16))) uint16_t tile[ROWS][CB + 8];
    __shared__ float part[4][ROWS * RANK];

    const int t = threadIdx.x, lane = t % 64, wave = t / 64;
    const int rloc = t / 8, slot = t % 8;
    const int64_t row = int64_t(blockIdx.x) * ROWS + rloc;
    const bool live = row < a.M;
    const int64_t K = a.K;
    const int64_t c0 = int64_t(blockIdx.y) * CB;
    const int ng = int(min(int64_t(CB), K - c0) / 64);  // 64-groups in this block
    const uint16_t* xr = a.x + (live ? row : 0) * a.ldx;

    float v[8][8];
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        if (live && g < ng) load8(xr + c0 + g * 64 + slot * 8, v[g]);
        else
            for (int j = 0; j < 8; ++j) v[g][j] = 0.0f;
    }
    if (a.stats && live) {
        const float2 st = a.stats[row];
#pragma unroll
        for (int g = 0; g < 8; ++g) {
            if (g >= ng) break;
            const int64_t col = c0 + g * 64 + slot * 8;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                float n = (v[g][j] - st.x) * st.y;
                if (a.ln_w) n = n * a.ln_w[col + j];
                if (a.ln_b) n = n + a.ln_b[col + j];
                if (a.mod_scale) n = n * (1.0f + a.mod_scale[col + j]);
                if (a.mod_shift) n = n + a.mod_shift[col + j];
                v[g][j] = bf16_to_f32(f32_to_bf16(n));
            }
        }
    }
    const float qmax = a.unsigned_q ? 15.0f : 7.0f;
    const float qlo = a.unsigned_q ? 0.0f : -8.0f;
#pragma unroll
    for (int g = 0; g < 8; ++g) {
        if (g >= ng) break;
        const int64_t col = c0 + g * 64 + slot * 8;
        uint16_t vb[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) vb[j] = f32_to_bf16(v[g][j]);
        const uint4 packed = make_uint4(vb[0] | (uint32_t(vb[1]) << 16), vb[2] | (uint32_t(vb[3]) << 16),
                                        vb[4] | (uint32_t(vb[5]) << 16), vb[6] | (uint32_t(vb[7]) << 16));
        *reinterpret_cast<uint4*>(&tile[rloc][g * 64 + slot * 8]) = packed;
        if (a.v_out && live) *reinterpret_cast<uint4*>(a.v_out + row * K + col) = packed;
        float u[8];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            u[j] = (v[g][j] + a.qshift) / bf16_to_f32(a.smooth[col + j]);
            amax = fmaxf(amax, fabsf(u[j]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
        const uint16_t sb = f32_to_bf16(amax / qmax);
        const float sc = bf16_to_f32(sb);
        float qv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float r = sc > 0.0f ? __builtin_rintf(u[j] / sc) : 0.0f;
            qv[j] = live ? fminf(fmaxf(r, qlo), qmax) + 0.0f : 0.0f;  // + 0 turns -0 into +0
        }
        uint32_t w0 = 0, w1 = 0;
        w0 = __builtin_amdgcn_cvt_pk_fp8_f32(qv[0], qv[1], w0, false);
        w0 = __builtin_amdgcn_cvt_pk_fp8_f32(qv[2], qv[3], w0, true);
        w1 = __builtin_amdgcn_cvt_pk_fp8_f32(qv[4], qv[5], w1, false);
        w1 = __builtin_amdgcn_cvt_pk_fp8_f32(qv[6], qv[7], w1, true);
        if (row < a.Mp) {
            *reinterpret_cast<uint2*>(a.q + row * K + col) = make_uint2(w0, w1);
            if (slot == 0) a.ascales[(col / 64) * a.Mp + row] = live ? sb : uint16_t(0);
        }
    }
    if (!a.pdt) return;
    __syncthreads();
    // wave w: k = 128 w .. 128 w + 127 of this block, 16 per MFMA; A = v rows (lane % 32), B = proj_down^T rows r
    f32x16 acc = {};
    const int kw = wave * 128;
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        const int kk = kw + s * 16 + 8 * (lane / 32);
        if (kw + s * 16 >= ng * 64) break;
        const bf16x8 av = *reinterpret_cast<const bf16x8*>(&tile[lane % 32][kk]);
        const bf16x8 bv = *reinterpret_cast<const bf16x8*>(a.pdt + int64_t(lane % 32) * K + c0 + kk);
        acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) part[wave][(8 * (i / 4) + 4 * (lane / 32) + (i % 4)) * RANK + lane % 32] = acc[i];
    __syncthreads();
    float* dst = a.lora + int64_t(blockIdx.y) * a.Mp * RANK;
    for (int e = t; e < ROWS * RANK; e += 256) {
        const int64_t r = int64_t(blockIdx.x) * ROWS + e / RANK;
        if (r < a.Mp) dst[r * RANK + e % RANK] = r < a.M ? (part[0][e] + part[1][e]) + (part[2][e] + part[3][e]) : 0.0f;
    }
}

__global__ void lora_sum_kernel(const float* part, int nb, int64_t n, float* out) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float s = part[i];
    for (int b = 1; b < nb; ++b) s = s + part[int64_t(b) * n + i];
    out[i] = s;
}

}  // namespace

extern "C" int64_t wdl_act_quant_workspace_floats(int64_t Mp, int64_t K) {
    const int64_t nb = (K + CB - 1) / CB;
    return (nb > 1 ? nb * Mp * RANK : 0) + 2 * Mp;
}

extern "C" int wdl_act_quant_w4(const void* x, int64_t ldx, int64_t M, int64_t K, const void* smooth, float qshift,
                                int unsigned_q, const void* proj_down_t, int64_t rank, void* q, void* ascales,
                                float* lora, int64_t Mp, const float* mod_shift, const float* mod_scale,
                                const float* ln_w, const float* ln_b, int ln, float eps, void* v_out,
                                float* workspace, hipStream_t stream) {
    if (M < 0 || K <= 0 || K % 64 || Mp < M || Mp % ROWS || ldx < K)
        return fail(WDL_EINVAL, "act_quant_w4: bad shape M=%lld K=%lld Mp=%lld ldx=%lld", (long long)M,
                    (long long)K, (long long)Mp, (long long)ldx);
    if (ln && K > 64 * 8 * MAXCH) return fail(WDL_EINVAL, "act_quant_w4: LayerNorm rows above 4096");
    if (proj_down_t && rank != RANK) return fail(WDL_EINVAL, "act_quant_w4: rank %lld != 32", (long long)rank);
    if (!x || !smooth || !q || !ascales || (proj_down_t && !lora) || !workspace)
        return fail(WDL_EINVAL, "act_quant_w4: null pointer");
    if ((reinterpret_cast<uintptr_t>(x) | (ldx * 2)) % 16)
        return fail(WDL_EINVAL, "act_quant_w4: x rows must be 16-byte aligned");
    if (Mp == 0) return WDL_OK;
    const int nb = int((K + CB - 1) / CB);
    float2* stats = reinterpret_cast<float2*>(workspace + (nb > 1 ? int64_t(nb) * Mp * RANK : 0));
    if (ln && M > 0) {
        row_stats_kernel<<<unsigned((M + 3) / 4), 256, 0, stream>>>(static_cast<const uint16_t*>(x), ldx, M, K, eps,
                                                                    stats);
        int rc = check_launch("act_quant_w4 row_stats");
        if (rc) return rc;
    }
    QuantArgs a{static_cast<const uint16_t*>(x), ldx, M, Mp, K, static_cast<const uint16_t*>(smooth), qshift,
                unsigned_q, static_cast<const uint16_t*>(proj_down_t), static_cast<uint8_t*>(q),
                static_cast<uint16_t*>(ascales), nb > 1 ? workspace : lora, ln ? stats : nullptr, mod_shift,
                mod_scale, ln_w, ln_b, static_cast<uint16_t*>(v_out)};
    quant_kernel<<<dim3(unsigned(Mp / ROWS), unsigned(nb)), 256, 0, stream>>>(a);
    int rc = check_launch("act_quant_w4 quant");
    if (rc || !proj_down_t || nb == 1) return rc;
    const int64_t n = Mp * RANK;
    lora_sum_kernel<<<unsigned((n + 255) / 256), 256, 0, stream>>>(workspace, nb, n, lora);
    return check_launch("act_quant_w4 lora_sum");
}
