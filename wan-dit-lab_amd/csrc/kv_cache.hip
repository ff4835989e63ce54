// FP8 KV-cache append: keys and values [B, n, H, D] (any strides, fp32/fp16/bf16) quantized row by row straight
// into the persistent cache [B, capacity, H, D] e4m3 at token offset `at`, with one fp32 scale per (token, head)
// in [B, capacity, H, 1]. Row rule (quantize_rows): scale = max(max|x|, 1e-12) / 448, value = e4m3(x / scale),
// both divisions IEEE, the fp8 rounding to nearest even. HBM-bound: one pass over the row, kept in registers.
#include "wdl_common.h"

namespace {

using namespace wdl;

struct Rows {
    const void* x;
    int64_t s0, s1, s2, s3;  // element strides of x
    uint8_t* cache;
    float* scale;
};

template <typename T>
struct Elem {
    using raw = uint16_t;
};
template <>
struct Elem<float> {
    using raw = float;
};

template <typename T>
__device__ __forceinline__ float to_f32(typename Elem<T>::raw r);
template <>
__device__ __forceinline__ float to_f32<float>(float r) { return r; }
template <>
__device__ __forceinline__ float to_f32<uint16_t>(uint16_t r) { return bf16_to_f32(r); }
template <>
__device__ __forceinline__ float to_f32<half_tag>(uint16_t r) { return f16_to_f32(r); }

// Lanes of one row: G (a power of two <= 64); each lane holds E elements d = lane + G * j in registers.
template <typename T, int G, int E>
__global__ __launch_bounds__(256) void kv_append_kernel(Rows k, Rows v, int64_t n, int64_t H, int64_t D,
                                                        int64_t rows, int64_t capacity, int64_t at) {
    const Rows& r = blockIdx.y == 0 ? k : v;
    const int lane = threadIdx.x % G;
    const int64_t row = int64_t(blockIdx.x) * (256 / G) + threadIdx.x / G;
    const bool live = row < rows;
    const int64_t h = row % H, tok = (row / H) % n, b = row / (H * n);
    const typename Elem<T>::raw* x = static_cast<const typename Elem<T>::raw*>(r.x);
    const int64_t base = b * r.s0 + tok * r.s1 + h * r.s2;
    float val[E];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int64_t d = lane + int64_t(G) * j;
        val[j] = (live && d < D) ? to_f32<T>(x[base + d * r.s3]) : 0.0f;
        amax = fmaxf(amax, fabsf(val[j]));
    }
    amax = group_max<G>(amax);
    const float scale = fmaxf(amax, 1e-12f) / 448.0f;
    if (!live) return;
    const int64_t target = (b * capacity + at + tok) * H + h;
    uint8_t* out = r.cache + target * D;
#pragma unroll
    for (int j = 0; j < E; ++j) {
        const int64_t d = lane + int64_t(G) * j;
        if (d < D) out[d] = f32_to_e4m3(val[j] / scale);
    }
    if (lane == 0) r.scale[target] = scale;
}

// Rows of D = 128 two-byte elements, unit element stride and 16-byte aligned: 16 lanes per row, lane l loads
// elements 8l .. 8l + 7 with one 16-byte load and stores their 8 codes with one 8-byte store (the same values as
// kv_append_kernel: the row maximum does not depend on the lane map).
template <typename T>
__global__ __launch_bounds__(256) void kv_append_vec_kernel(Rows k, Rows v, int64_t n, int64_t H, int64_t rows,
                                                            int64_t capacity, int64_t at) {
    const Rows& r = blockIdx.y == 0 ? k : v;
    const int lane = threadIdx.x % 16;
    const int64_t row = int64_t(blockIdx.x) * 16 + threadIdx.x / 16;
    const bool live = row < rows;
    const int64_t h = row % H, tok = (row / H) % n, b = row / (H * n);
    uint4 raw = make_uint4(0, 0, 0, 0);
    if (live)
        raw = *reinterpret_cast<const uint4*>(static_cast<const uint16_t*>(r.x) + b * r.s0 + tok * r.s1 + h * r.s2 +
                                              8 * lane);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
    float val[8];
    float amax = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        val[2 * j] = to_f32<T>(uint16_t(w[j] & 0xffffu));
        val[2 * j + 1] = to_f32<T>(uint16_t(w[j] >> 16));
        amax = fmaxf(amax, fmaxf(fabsf(val[2 * j]), fabsf(val[2 * j + 1])));
    }
    amax = group_max<16>(amax);
    const float scale = fmaxf(amax, 1e-12f) / 448.0f;
    if (!live) return;
    const int64_t target = (b * capacity + at + tok) * H + h;
    // the IEEE quotients val / scale through the reciprocal (div_rn: correctly rounded wherever |quotient| >=
    // 2^-126; below that every value encodes to a zero of the quotient's sign, which div_rn keeps)
    const float rs = 1.0f / scale;
    uint32_t c[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
        c[j] = e4m3x4(div_rn(val[4 * j], scale, rs), div_rn(val[4 * j + 1], scale, rs),
                      div_rn(val[4 * j + 2], scale, rs), div_rn(val[4 * j + 3], scale, rs));
    *reinterpret_cast<uint2*>(r.cache + target * 128 + 8 * lane) = make_uint2(c[0], c[1]);
    if (lane == 0) r.scale[target] = scale;
}

template <typename T, int G, int E>
void launch_rows(const Rows& k, const Rows& v, int two, int64_t n, int64_t H, int64_t D, int64_t rows,
                 int64_t capacity, int64_t at, hipStream_t stream) {
    dim3 grid(unsigned((rows + 256 / G - 1) / (256 / G)), unsigned(two));
    kv_append_kernel<T, G, E><<<grid, 256, 0, stream>>>(k, v, n, H, D, rows, capacity, at);
}

// D up to 64 * 16 = 1024 elements per row
template <typename T>
int dispatch(const Rows& k, const Rows& v, int two, int64_t n, int64_t H, int64_t D, int64_t rows,
             int64_t capacity, int64_t at, hipStream_t stream) {
    const auto vec_ok = [](const Rows& r) {
        return r.s3 == 1 && (reinterpret_cast<uintptr_t>(r.x) | ((r.s0 | r.s1 | r.s2) * 2)) % 16 == 0 &&
               reinterpret_cast<uintptr_t>(r.cache) % 8 == 0;
    };
    if (sizeof(typename Elem<T>::raw) == 2 && D == 128 && vec_ok(k) && vec_ok(v)) {
        const dim3 grid(unsigned((rows + 15) / 16), unsigned(two));
        kv_append_vec_kernel<T><<<grid, 256, 0, stream>>>(k, v, n, H, rows, capacity, at);
    } else if (D <= 64) {
        launch_rows<T, 16, 4>(k, v, two, n, H, D, rows, capacity, at, stream);
    } else if (D <= 128) {
        launch_rows<T, 16, 8>(k, v, two, n, H, D, rows, capacity, at, stream);
    } else if (D <= 256) {
        launch_rows<T, 32, 8>(k, v, two, n, H, D, rows, capacity, at, stream);
    } else if (D <= 1024) {
        launch_rows<T, 64, 16>(k, v, two, n, H, D, rows, capacity, at, stream);
    } else {
        return fail(WDL_EINVAL, "kv_append_fp8: head_dim %lld > 1024", (long long)D);
    }
    return check_launch("kv_append_fp8");
}

int dispatch_dtype(int dtype, const Rows& k, const Rows& v, int two, int64_t n, int64_t H, int64_t D, int64_t rows,
                   int64_t capacity, int64_t at, hipStream_t stream) {
    switch (dtype) {
        case WDL_F32: return dispatch<float>(k, v, two, n, H, D, rows, capacity, at, stream);
        case WDL_BF16: return dispatch<uint16_t>(k, v, two, n, H, D, rows, capacity, at, stream);
        case WDL_F16: return dispatch<half_tag>(k, v, two, n, H, D, rows, capacity, at, stream);
        default: return fail(WDL_EINVAL, "kv_append_fp8: unsupported dtype %d", dtype);
    }
}

}  // namespace

extern "C" int wdl_kv_append_fp8(const void* k, int k_dtype, const int64_t* k_strides, const void* v, int v_dtype,
                                 const int64_t* v_strides, int64_t B, int64_t n, int64_t H, int64_t D, void* cache_k,
                                 float* cache_ks, void* cache_v, float* cache_vs, int64_t capacity, int64_t at,
                                 hipStream_t stream) {
    if (B < 0 || n < 0 || H < 0 || D < 1) return fail(WDL_EINVAL, "kv_append_fp8: bad shape");
    if (at < 0 || at + n > capacity) return fail(WDL_EINVAL, "kv_append_fp8: write [%lld, %lld) exceeds capacity %lld",
                                                 (long long)at, (long long)(at + n), (long long)capacity);
    if (!k || !v || !cache_k || !cache_ks || !cache_v || !cache_vs || !k_strides || !v_strides)
        return fail(WDL_EINVAL, "kv_append_fp8: null pointer");
    const int64_t rows = B * n * H;
    if (rows == 0) return WDL_OK;
    Rows rk{k, k_strides[0], k_strides[1], k_strides[2], k_strides[3], static_cast<uint8_t*>(cache_k), cache_ks};
    Rows rv{v, v_strides[0], v_strides[1], v_strides[2], v_strides[3], static_cast<uint8_t*>(cache_v), cache_vs};
    if (k_dtype == v_dtype) return dispatch_dtype(k_dtype, rk, rv, 2, n, H, D, rows, capacity, at, stream);
    int rc = dispatch_dtype(k_dtype, rk, rk, 1, n, H, D, rows, capacity, at, stream);
    if (rc != WDL_OK) return rc;
    return dispatch_dtype(v_dtype, rv, rv, 1, n, H, D, rows, capacity, at, stream);
}
