// The general 3D RoPE rotation of wan_dit_lab::rope3d_rotate (kernels/rope_triton.py:14-81): any batch with one
// (f, h, w) grid per sample, any element strides, fp16 / bf16 / fp32 / fp64 input and output, fp32 or fp64 tables,
// the inverse rotation for the backward pass. The block's own path uses the fused Q/K RMSNorm + RoPE kernel
// (qk_rope.hip); this one is the standalone operator.
//
// One thread per (sample, token, head, pair): pair p of token i turns by the angle of its axis (time pairs first:
// start + i // (h w); then height (i // w) % h; then width i % w), (e, o) -> (e c - o s, o c + e s), s negated when
// inverse. Arithmetic in fp64 when the input or the table is fp64, else fp32, each product rounded (the library is
// built without contraction); fp16 / bf16 results pass through fp32 (torch's fp64 -> half casts do); tokens past
// f h w are copied through the same conversions. The output is contiguous [B, L, H, dim].
#include "wdl_common.h"

namespace {

using namespace wdl;

constexpr int MAX_BATCH = 64;

struct RopeArgs {
    const void* x;
    int x_dtype;
    int64_t xs[4];
    const void* freq;
    int freq_dtype;
    int64_t fs[3];
    void* out;
    int out_dtype;
    int64_t L, H, pairs, total;
    int64_t start;
    int inverse;
    int grids[MAX_BATCH][3];
};

__device__ __forceinline__ double load_f64(const void* p, int dtype, int64_t i) {
    switch (dtype) {
        case WDL_F64: return static_cast<const double*>(p)[i];
        case WDL_F32: return static_cast<const float*>(p)[i];
        case WDL_F16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
        default: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
}

__device__ __forceinline__ float load_f32(const void* p, int dtype, int64_t i) {
    switch (dtype) {
        case WDL_F32: return static_cast<const float*>(p)[i];
        case WDL_F16: return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
        default: return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
    }
}

// a result of the fp32 path to the output type
__device__ __forceinline__ void store_f32(void* p, int dtype, int64_t i, float v) {
    switch (dtype) {
        case WDL_F64: static_cast<double*>(p)[i] = v; break;
        case WDL_F32: static_cast<float*>(p)[i] = v; break;
        case WDL_F16: static_cast<uint16_t*>(p)[i] = f32_to_f16(v); break;
        default: static_cast<uint16_t*>(p)[i] = f32_to_bf16(v); break;
    }
}

// a result of the fp64 path: fp16 / bf16 through fp32, as torch casts them
__device__ __forceinline__ void store_f64(void* p, int dtype, int64_t i, double v) {
    if (dtype == WDL_F64) static_cast<double*>(p)[i] = v;
    else store_f32(p, dtype, i, float(v));
}

template <bool F64>
__global__ __launch_bounds__(256) void rope3d_kernel(RopeArgs a) {
    const int64_t idx = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (idx >= a.total) return;
    const int64_t p = idx % a.pairs, hd = (idx / a.pairs) % a.H, tok = (idx / (a.pairs * a.H)) % a.L;
    const int64_t b = idx / (a.pairs * a.H * a.L);
    const int f = a.grids[b][0], gh = a.grids[b][1], gw = a.grids[b][2];
    const int64_t spatial = a.pairs / 3, tp = a.pairs - 2 * spatial;
    const int64_t xi = b * a.xs[0] + tok * a.xs[1] + hd * a.xs[2] + 2 * p * a.xs[3];
    const int64_t oi = ((b * a.L + tok) * a.H + hd) * (2 * a.pairs) + 2 * p;
    const bool rotate = tok < int64_t(f) * gh * gw;
    int64_t pos = 0;
    if (rotate) pos = p < tp ? a.start + tok / (int64_t(gh) * gw) : (p < tp + spatial ? (tok / gw) % gh : tok % gw);
    const int64_t fi = pos * a.fs[1] + p * a.fs[2];
    if (F64) {
        const double e = load_f64(a.x, a.x_dtype, xi), o = load_f64(a.x, a.x_dtype, xi + a.xs[3]);
        double re = e, ro = o;
        if (rotate) {
            const double c = load_f64(a.freq, a.freq_dtype, fi);
            double s = load_f64(a.freq, a.freq_dtype, a.fs[0] + fi);
            if (a.inverse) s = -s;
            re = e * c - o * s;
            ro = o * c + e * s;
        }
        store_f64(a.out, a.out_dtype, oi, re);
        store_f64(a.out, a.out_dtype, oi + 1, ro);
    } else {
        const float e = load_f32(a.x, a.x_dtype, xi), o = load_f32(a.x, a.x_dtype, xi + a.xs[3]);
        float re = e, ro = o;
        if (rotate) {
            const float c = load_f32(a.freq, a.freq_dtype, fi);
            float s = load_f32(a.freq, a.freq_dtype, a.fs[0] + fi);
            if (a.inverse) s = -s;
            re = e * c - o * s;
            ro = o * c + e * s;
        }
        store_f32(a.out, a.out_dtype, oi, re);
        store_f32(a.out, a.out_dtype, oi + 1, ro);
    }
}

bool valid_dtype(int d) { return d == WDL_F32 || d == WDL_F16 || d == WDL_BF16 || d == WDL_F64; }

}  // namespace

extern "C" int wdl_rope3d_rotate(const void* x, int x_dtype, const int64_t* x_strides, const void* freq,
                                 int freq_dtype, const int64_t* freq_strides, int64_t positions, int64_t B, int64_t L,
                                 int64_t H, int64_t dim, const int32_t* grids, int64_t start, int inverse, void* out,
                                 int out_dtype, hipStream_t stream) {
    if (B < 1 || B > MAX_BATCH || L < 0 || H < 1 || dim < 2 || dim % 2 || positions < 1 || start < 0)
        return fail(WDL_EINVAL, "rope3d_rotate: bad shape B=%lld L=%lld H=%lld dim=%lld (batch 1..%d, even dim)",
                    (long long)B, (long long)L, (long long)H, (long long)dim, MAX_BATCH);
    if (!valid_dtype(x_dtype) || !valid_dtype(out_dtype) || (freq_dtype != WDL_F32 && freq_dtype != WDL_F64))
        return fail(WDL_EINVAL, "rope3d_rotate: dtypes: input and output fp16/bf16/fp32/fp64, tables fp32/fp64");
    if (!x_strides || !freq_strides || !grids || (L > 0 && (!x || !freq || !out)))
        return fail(WDL_EINVAL, "rope3d_rotate: null pointer");
    const int64_t pairs = dim / 2, spatial = pairs / 3;
    for (int64_t b = 0; b < B; ++b) {
        const int64_t f = grids[3 * b], h = grids[3 * b + 1], w = grids[3 * b + 2];
        if (f < 0 || h < 1 || w < 1 || f * h * w > L || start + f > positions ||
            (spatial > 0 && (h > positions || w > positions)))
            return fail(WDL_EINVAL, "rope3d_rotate: grid %lld of (%lld, %lld, %lld) exceeds the sequence or the table",
                        (long long)b, (long long)f, (long long)h, (long long)w);
    }
    if (L == 0) return WDL_OK;
    RopeArgs a{};
    a.x = x, a.x_dtype = x_dtype, a.freq = freq, a.freq_dtype = freq_dtype, a.out = out, a.out_dtype = out_dtype;
    for (int i = 0; i < 4; ++i) a.xs[i] = x_strides[i];
    for (int i = 0; i < 3; ++i) a.fs[i] = freq_strides[i];
    a.L = L, a.H = H, a.pairs = pairs, a.total = B * L * H * pairs, a.start = start, a.inverse = inverse ? 1 : 0;
    for (int64_t b = 0; b < B; ++b)
        for (int i = 0; i < 3; ++i) a.grids[b][i] = grids[3 * b + i];
    const unsigned blocks = unsigned((a.total + 255) / 256);
    if (x_dtype == WDL_F64 || freq_dtype == WDL_F64) rope3d_kernel<true><<<blocks, 256, 0, stream>>>(a);
    else rope3d_kernel<false><<<blocks, 256, 0, stream>>>(a);
    return check_launch("rope3d_rotate");
}
