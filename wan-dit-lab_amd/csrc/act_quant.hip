// Per-token, per-64-channel activation quantizer of the W4A4 linears, optionally fused with the LayerNorm and the
// adaLN modulation that precede it, and with the down projection of the low-rank branch.
//
// For rows m < M of x (bf16 [M, K], row stride ldx):
//   v     = x                                           (plain), or
//   v     = bf16( LN(x)[*w + b] * (1 + mod_scale) + mod_shift )   (fused; fp32 math, one rounding)
//   u     = (v + qshift) / smooth                       (IEEE fp32)
//   scale = bf16( max_{64 group} |u| / qmax )           (qmax 7 signed, 15 unsigned)
//   q     = clamp(rint(u / scale))                      (0 where scale is 0)
//   lora  = v . proj_down                               (bf16 MFMA, fp32 sums)
// Outputs: q as e4m3 codes of the integer values (exact), one byte per value [Mp, K] (rows >= M zero);
// ascales bf16 [K/64, Mp]; lora fp32 [Mp, r] (r = 32). LN statistics use a fixed reduction order: 8 column
// slots per row, each summing its 8-wide chunks group by group, combined by an xor butterfly (4, 2, 1).
//
// One workgroup of 256 threads per 32 rows; thread t owns row t/8 and the 8 columns (t%8)*8.. of each group.
#include "wdl_common.h"

namespace {

using namespace wdl;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int ROWS = 32;
constexpr int RANK = 32;

struct QuantArgs {
    const uint16_t* x;
    int64_t ldx;
    int64_t M, Mp, K;
    const uint16_t* smooth;    // bf16 [K]
    float qshift;
    int unsigned_q;
    const uint16_t* pdt;       // bf16 [RANK, K] (proj_down transposed), may be null (no lora)
    uint8_t* q;                // [Mp, K]
    uint16_t* ascales;         // [K/64, Mp]
    float* lora;               // [Mp, RANK]
    // fused LayerNorm + modulation (ln != 0)
    int ln;
    const float* mod_shift;    // fp32 [K] or null
    const float* mod_scale;    // fp32 [K] or null (used as 1 + scale)
    const float* ln_w;         // fp32 [K] or null
    const float* ln_b;         // fp32 [K] or null
    float eps;
    uint16_t* v_out;           // bf16 [M, K] debug copy of v, or null
};

__device__ __forceinline__ void load8(const uint16_t* p, float* f) {
    uint4 raw = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = __uint_as_float(w[j] << 16);
        f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
}

// sum over the row in the fixed order: per thread g outer, j inner; then butterfly across the 8 slots
__device__ __forceinline__ float slot_combine(float s) {
    s = s + __shfl_xor(s, 4, 8);
    s = s + __shfl_xor(s, 2, 8);
    s = s + __shfl_xor(s, 1, 8);
    return s;
}

__global__ __launch_bounds__(256) void act_quant_kernel(QuantArgs a) {
    __shared__ uint16_t tile[ROWS][64 + 8];     // v of the current group, bf16, padded rows
    __shared__ float part[4][ROWS * RANK];      // per-wave lora partials

    const int t = threadIdx.x;
    const int rloc = t / 8, slot = t % 8;
    const int64_t row = int64_t(blockIdx.x) * ROWS + rloc;
    const bool live = row < a.M;
    const int64_t K = a.K;
    const int G = int(K / 64);
    const uint16_t* xr = a.x + (live ? row : 0) * a.ldx;

    float mean = 0.0f, rstd = 1.0f;
    if (a.ln) {
        float s = 0.0f;
        for (int g = 0; g < G; ++g) {
            float f[8];
            if (live) load8(xr + g * 64 + slot * 8, f);
            else
                for (int j = 0; j < 8; ++j) f[j] = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) s = s + f[j];
        }
        s = slot_combine(s);
        mean = s / float(K);
        float ss = 0.0f;
        for (int g = 0; g < G; ++g) {
            float f[8];
            if (live) load8(xr + g * 64 + slot * 8, f);
            else
                for (int j = 0; j < 8; ++j) f[j] = 0.0f;
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float d = f[j] - mean;
                ss = ss + d * d;
            }
        }
        ss = slot_combine(ss);
        const float var = ss / float(K);
        rstd = 1.0f / sqrtf(var + a.eps);  // sqrtf lowers to the correctly rounded sequence
    }

    const int wave = t / 64, lane = t % 64;
    f32x16 acc = {};
    const float qmax = a.unsigned_q ? 15.0f : 7.0f;
    const float qlo = a.unsigned_q ? 0.0f : -8.0f;

    for (int g = 0; g < G; ++g) {
        const int64_t col = int64_t(g) * 64 + slot * 8;
        float v[8];
        if (live) {
            load8(xr + col, v);
            if (a.ln) {
#pragma unroll
                for (int j = 0; j < 8; ++j) {
                    float n = (v[j] - mean) * rstd;
                    if (a.ln_w) n = n * a.ln_w[col + j];
                    if (a.ln_b) n = n + a.ln_b[col + j];
                    if (a.mod_scale) n = n * (1.0f + a.mod_scale[col + j]);
                    if (a.mod_shift) n = n + a.mod_shift[col + j];
                    v[j] = bf16_to_f32(f32_to_bf16(n));
                }
            }
        } else {
#pragma unroll
            for (int j = 0; j < 8; ++j) v[j] = 0.0f;
        }
        // stage v (bf16) for the low-rank MFMA, and the debug copy
        uint16_t vb[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) vb[j] = f32_to_bf16(v[j]);
        uint4 packed = make_uint4(vb[0] | (uint32_t(vb[1]) << 16), vb[2] | (uint32_t(vb[3]) << 16),
                                  vb[4] | (uint32_t(vb[5]) << 16), vb[6] | (uint32_t(vb[7]) << 16));
        *reinterpret_cast<uint4*>(&tile[rloc][slot * 8]) = packed;
        if (a.v_out && live) *reinterpret_cast<uint4*>(a.v_out + row * K + col) = packed;

        // quantize
        float u[8];
        float amax = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            u[j] = (v[j] + a.qshift) / bf16_to_f32(a.smooth[col + j]);
            amax = fmaxf(amax, fabsf(u[j]));
        }
        amax = fmaxf(amax, __shfl_xor(amax, 4, 8));
        amax = fmaxf(amax, __shfl_xor(amax, 2, 8));
        amax = fmaxf(amax, __shfl_xor(amax, 1, 8));
        const uint16_t sb = f32_to_bf16(amax / qmax);
        const float sc = bf16_to_f32(sb);
        uint32_t w0 = 0, w1 = 0;
        float qv[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            float r = sc > 0.0f ? __builtin_rintf(u[j] / sc) : 0.0f;
            qv[j] = fminf(fmaxf(r, qlo), qmax) + 0.0f;  // + 0 turns -0 into +0: one code per integer
        }
        if (!live) {
#pragma unroll
            for (int j = 0; j < 8; ++j) qv[j] = 0.0f;
        }
        w0 = __builtin_amdgcn_cvt_pk_fp8_f32(qv[0], qv[1], w0, false);
        w0 = __builtin_amdgcn_cvt_pk_fp8_f32(qv[2], qv[3], w0, true);
        w1 = __builtin_amdgcn_cvt_pk_fp8_f32(qv[4], qv[5], w1, false);
        w1 = __builtin_amdgcn_cvt_pk_fp8_f32(qv[6], qv[7], w1, true);
        if (row < a.Mp) {
            *reinterpret_cast<uint2*>(a.q + row * K + col) = make_uint2(w0, w1);
            if (slot == 0) a.ascales[int64_t(g) * a.Mp + row] = live ? sb : uint16_t(0);
        }
        __syncthreads();
        if (a.pdt) {
            // wave w: k = 16w .. 16w+15 of this group. A = v rows (lane: row lane%32, k 8*(lane/32)..+7),
            // B = proj_down^T rows r = lane%32.
            const int kk = wave * 16 + 8 * (lane / 32);
            bf16x8 av = *reinterpret_cast<const bf16x8*>(&tile[lane % 32][kk]);
            bf16x8 bv = *reinterpret_cast<const bf16x8*>(a.pdt + int64_t(lane % 32) * K + int64_t(g) * 64 + kk);
            acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(av, bv, acc, 0, 0, 0);
        }
        __syncthreads();
    }
    if (!a.pdt) return;
    // acc: lane holds r = lane%32 (column), rows 8*(i/4) + 4*(lane/32) + i%4
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        const int m = 8 * (i / 4) + 4 * (lane / 32) + (i % 4);
        part[wave][m * RANK + lane % 32] = acc[i];
    }
    __syncthreads();
    for (int e = t; e < ROWS * RANK; e += 256) {
        const int m = e / RANK;
        const int64_t r = int64_t(blockIdx.x) * ROWS + m;
        if (r < a.Mp) {
            const float s = (part[0][e] + part[1][e]) + (part[2][e] + part[3][e]);
            a.lora[r * RANK + e % RANK] = (r < a.M) ? s : 0.0f;
        }
    }
}

}  // namespace

extern "C" int wdl_act_quant_w4(const void* x, int64_t ldx, int64_t M, int64_t K, const void* smooth, float qshift,
                                int unsigned_q, const void* proj_down_t, int64_t rank, void* q, void* ascales,
                                float* lora, int64_t Mp, const float* mod_shift, const float* mod_scale,
                                const float* ln_w, const float* ln_b, int ln, float eps, void* v_out,
                                hipStream_t stream) {
    if (M < 0 || K <= 0 || K % 64 || Mp < M || Mp % ROWS || ldx < K)
        return fail(WDL_EINVAL, "act_quant_w4: bad shape M=%lld K=%lld Mp=%lld ldx=%lld", (long long)M,
                    (long long)K, (long long)Mp, (long long)ldx);
    if (proj_down_t && rank != RANK) return fail(WDL_EINVAL, "act_quant_w4: rank %lld != 32", (long long)rank);
    if (!x || !smooth || !q || !ascales || (proj_down_t && !lora))
        return fail(WDL_EINVAL, "act_quant_w4: null pointer");
    if ((reinterpret_cast<uintptr_t>(x) | (ldx * 2)) % 16)
        return fail(WDL_EINVAL, "act_quant_w4: x rows must be 16-byte aligned");
    if (Mp == 0) return WDL_OK;
    QuantArgs a{static_cast<const uint16_t*>(x), ldx, M, Mp, K, static_cast<const uint16_t*>(smooth), qshift,
                unsigned_q, static_cast<const uint16_t*>(proj_down_t), static_cast<uint8_t*>(q),
                static_cast<uint16_t*>(ascales), lora, ln, mod_shift, mod_scale, ln_w, ln_b, eps,
                static_cast<uint16_t*>(v_out)};
    act_quant_kernel<<<unsigned(Mp / ROWS), 256, 0, stream>>>(a);
    return check_launch("act_quant_w4");
}
