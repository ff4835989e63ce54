// FP8 (E4M3FN) quantization of linear-layer operands (src/wan_dit_lab/quantization/fp8.py):
//   per row    (quantize_rows, fp8.py:37-41): scale[m] = max(max_k |x[m][k]|, 1e-12) / 448, q = e4m3(x / scale)
//   per tensor (quantize,      fp8.py:14-17): scale    = max(max    |x|,       1e-12) / 448, q = e4m3(x / scale)
// x is bf16 or fp32 [M, K] (row stride ldx); q is [Mp, K] bytes (rows M..Mp-1 zero, the padding the FP8 GEMM
// tiles need), scale fp32 [Mp] (rows: padding rows 0) or [1]. The quotient is IEEE fp32 and the conversion is the
// hardware's round-to-nearest-even e4m3 conversion (torch's; the largest |x| lands on 448). Per tensor with a bf16
// x, the reference's X / scale divides by a 0-d fp32 tensor, which does not promote the bf16 result: the quotient
// is rounded to bf16 before the e4m3 conversion (the per-row scale [..., 1] does promote: fp32 quotient there).
//
// rows:   one workgroup per row (4 waves from K = 2048 on, else 1), two passes over it (the maximum, then the codes;
//         the second pass reads the row back from cache), 16 bytes of bf16 per lane and load.
// tensor: pass 1 writes one partial maximum per workgroup to the workspace; pass 2 has every workgroup reduce
//         the partials (the same order in each: deterministic) and quantize its share. No atomics, no memory that
//         has to start zeroed.
#include "wdl_common.h"

namespace {

using namespace wdl;

constexpr float FP8_MAX = 448.0f;
constexpr int TBLOCKS = 512;  // workgroups of the per-tensor passes (at most)

// 4 consecutive values of a row as floats (16-byte loads of fp32, 8-byte of bf16)
template <typename T>
__device__ __forceinline__ void ld4(const T* p, float* f);
template <>
__device__ __forceinline__ void ld4<uint16_t>(const uint16_t* p, float* f) {
    const uint2 r = *reinterpret_cast<const uint2*>(p);
    f[0] = __uint_as_float(r.x << 16), f[1] = __uint_as_float(r.x & 0xffff0000u);
    f[2] = __uint_as_float(r.y << 16), f[3] = __uint_as_float(r.y & 0xffff0000u);
}
template <>
__device__ __forceinline__ void ld4<float>(const float* p, float* f) {
    const float4 r = *reinterpret_cast<const float4*>(p);
    f[0] = r.x, f[1] = r.y, f[2] = r.z, f[3] = r.w;
}

__device__ __forceinline__ uint32_t e4m3x4(const float* y) { return wdl::e4m3x4(y[0], y[1], y[2], y[3]); }

// 8 consecutive values of a row as floats (one 16-byte load of bf16, two of fp32)
template <typename T>
__device__ __forceinline__ void ld8(const T* p, float* f) {
    ld4<T>(p, f);
    ld4<T>(p + 4, f + 4);
}
template <>
__device__ __forceinline__ void ld8<uint16_t>(const uint16_t* p, float* f) {
    const uint4 r = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {r.x, r.y, r.z, r.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) f[2 * e] = __uint_as_float(w[e] << 16), f[2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
}

// One workgroup of WPR waves per row, 8 values per lane and step, two steps in flight: the row's maximum (lanes,
// then waves through LDS), then the codes from a second read of the row (from cache). The maximum is
// order-independent, so the result is the same for any WPR.
template <typename T, int WPR>
__global__ __launch_bounds__(64 * WPR) void rows_kernel(const T* x, int64_t ldx, int64_t M, int64_t K, uint8_t* q,
                                                        float* scale) {
    __shared__ float red[WPR];
    const int t = threadIdx.x;
    const int64_t row = blockIdx.x;
    constexpr int NT = 64 * WPR;
    uint2* qr = reinterpret_cast<uint2*>(q + row * K);
    const int64_t chunks = K / 8;
    if (row >= M) {  // padding rows of the GEMM tiles: zero codes, zero scale
        for (int64_t c = t; c < chunks; c += NT) qr[c] = make_uint2(0u, 0u);
        if (t == 0) scale[row] = 0.0f;
        return;
    }
    const T* xr = x + row * ldx;
    float amax = 0.0f;
    int64_t c = t;
    for (; c + NT < chunks; c += 2 * NT) {
        float f[8], g[8];
        ld8<T>(xr + 8 * c, f);
        ld8<T>(xr + 8 * (c + NT), g);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fmaxf(fabsf(f[e]), fabsf(g[e])));
    }
    if (c < chunks) {
        float f[8];
        ld8<T>(xr + 8 * c, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
    }
    amax = group_max<64>(amax);
    if (WPR > 1) {
        if (t % 64 == 0) red[t / 64] = amax;
        __syncthreads();
        amax = red[0];
#pragma unroll
        for (int w = 1; w < WPR; ++w) amax = fmaxf(amax, red[w]);
    }
    const float s = fmaxf(amax, 1e-12f) / FP8_MAX;
    if (t == 0) scale[row] = s;
    auto codes = [&](int64_t cc) {
        float f[8];
        ld8<T>(xr + 8 * cc, f);
#pragma unroll
        for (int e = 0; e < 8; ++e) f[e] = f[e] / s;
        qr[cc] = make_uint2(e4m3x4(f), e4m3x4(f + 4));
    };
    c = t;
    for (; c + NT < chunks; c += 2 * NT) {
        codes(c);
        codes(c + NT);
    }
    if (c < chunks) codes(c);
}

template <typename T>
__global__ __launch_bounds__(256) void tensor_max_kernel(const T* x, int64_t ldx, int64_t M, int64_t K,
                                                         float* partial) {
    __shared__ float red[4];
    const int64_t k8 = K / 8, n8 = M * k8, stride = int64_t(gridDim.x) * 256;
    float amax = 0.0f;
    int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    for (; i + stride < n8; i += 2 * stride) {  // two 16-byte loads of bf16 in flight
        float f[8], g[8];
        ld8<T>(x + (i / k8) * ldx + 8 * (i % k8), f);
        ld8<T>(x + ((i + stride) / k8) * ldx + 8 * ((i + stride) % k8), g);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fmaxf(fabsf(f[e]), fabsf(g[e])));
    }
    if (i < n8) {
        float f[8];
        ld8<T>(x + (i / k8) * ldx + 8 * (i % k8), f);
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(f[e]));
    }
    amax = group_max<64>(amax);
    if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = amax;
    __syncthreads();
    if (threadIdx.x == 0) partial[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
}

template <typename T>
__global__ __launch_bounds__(256) void tensor_quant_kernel(const T* x, int64_t ldx, int64_t M, int64_t Mp, int64_t K,
                                                           const float* partial, int nparts, uint8_t* q, float* scale) {
    __shared__ float red[4];
    float amax = 0.0f;
    for (int i = threadIdx.x; i < nparts; i += 256) amax = fmaxf(amax, partial[i]);
    amax = group_max<64>(amax);
    if (threadIdx.x % 64 == 0) red[threadIdx.x / 64] = amax;
    __syncthreads();
    const float s = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), 1e-12f) / FP8_MAX;
    if (blockIdx.x == 0 && threadIdx.x == 0) scale[0] = s;
    const int64_t k8 = K / 8, n8 = Mp * k8, stride = int64_t(gridDim.x) * 256;
    auto codes = [&](int64_t i) {
        const int64_t m = i / k8, c = i % k8;
        uint2 w = make_uint2(0u, 0u);
        if (m < M) {
            float f[8];
            ld8<T>(x + m * ldx + 8 * c, f);
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                f[e] = f[e] / s;
                if constexpr (sizeof(T) == 2) f[e] = bf16_to_f32(f32_to_bf16(f[e]));
            }
            w = make_uint2(e4m3x4(f), e4m3x4(f + 4));
        }
        reinterpret_cast<uint2*>(q + m * K)[c] = w;
    };
    int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    for (; i + stride < n8; i += 2 * stride) {
        codes(i);
        codes(i + stride);
    }
    if (i < n8) codes(i);
}

int tensor_blocks(int64_t M, int64_t K) {
    const int64_t n8 = M * (K / 8);
    const int64_t b = (n8 + 256 * 4 - 1) / (256 * 4);
    return int(b < 1 ? 1 : (b > TBLOCKS ? TBLOCKS : b));
}

template <typename T>
int quantize(const void* xv, int64_t ldx, int64_t M, int64_t K, int64_t Mp, int rows, void* q, float* scale,
             float* workspace, hipStream_t stream) {
    const T* x = static_cast<const T*>(xv);
    uint8_t* qb = static_cast<uint8_t*>(q);
    if (rows) {
        if (K >= 2048) rows_kernel<T, 4><<<unsigned(Mp), 256, 0, stream>>>(x, ldx, M, K, qb, scale);
        else rows_kernel<T, 1><<<unsigned(Mp), 64, 0, stream>>>(x, ldx, M, K, qb, scale);
        return check_launch("fp8_quantize rows");
    }
    const int nb = tensor_blocks(M, K);
    if (M > 0) {
        tensor_max_kernel<T><<<unsigned(nb), 256, 0, stream>>>(x, ldx, M, K, workspace);
        const int rc = check_launch("fp8_quantize tensor max");
        if (rc) return rc;
    }
    tensor_quant_kernel<T><<<unsigned(nb), 256, 0, stream>>>(x, ldx, M, Mp, K, workspace, M > 0 ? nb : 0, qb, scale);
    return check_launch("fp8_quantize tensor");
}

}  // namespace

extern "C" int64_t wdl_fp8_quantize_workspace_floats(int64_t M, int64_t K) { return tensor_blocks(M, K); }

extern "C" int wdl_fp8_quantize(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t Mp, int rows,
                                void* q, float* scale, float* workspace, hipStream_t stream) {
    if (M < 0 || K <= 0 || K % 16 || Mp < M || ldx < K)
        return fail(WDL_EINVAL, "fp8_quantize: bad shape M=%lld K=%lld Mp=%lld ldx=%lld", (long long)M, (long long)K,
                    (long long)Mp, (long long)ldx);
    if (x_dtype != WDL_BF16 && x_dtype != WDL_F32) return fail(WDL_EINVAL, "fp8_quantize: x must be bf16 or fp32");
    if (!x || !q || !scale || (!rows && !workspace)) return fail(WDL_EINVAL, "fp8_quantize: null pointer");
    const int64_t esz = x_dtype == WDL_F32 ? 4 : 2;
    if ((reinterpret_cast<uintptr_t>(x) | (ldx * esz) | reinterpret_cast<uintptr_t>(q)) % 16)
        return fail(WDL_EINVAL, "fp8_quantize: rows must be 16-byte aligned");
    if (Mp == 0) return WDL_OK;
    return x_dtype == WDL_F32 ? quantize<float>(x, ldx, M, K, Mp, rows, q, scale, workspace, stream)
                              : quantize<uint16_t>(x, ldx, M, K, Mp, rows, q, scale, workspace, stream);
}
