// Q/K RMSNorm over the whole row (all heads) and 3D RoPE, fused, plus Sage's per-thread int8 quantization of Q.
//
// qk_norm_rope: two waves per (row m, q or k), the row held in registers (bf16, row strides ldq / ldk, H heads of
// D = 128, H * D <= 4096):
//   rstd = 1 / sqrt(mean(x^2) + eps)     fp32; ordered sum: lane l owns the 8-value chunks c = l, l + 64, ... and
//                                       adds their squares value by value (the first wave's chunks, then the
//                                       second's), then an xor butterfly 32, 16, .., 1
//   n   = bf16(x * rstd);  w = bf16(n * weight)                                (models/rms_norm.py:12-13)
//   rot = bf16(w1 c - w2 s), bf16(w2 c + w1 s) on pairs (2p, 2p+1)             (models/rope.py:26-31)
// in the table's precision: fp32 for an fp32 table; for an fp64 table the products and differences are fp64 and the
// result is rounded to fp32, then to bf16 (torch's double -> bfloat16 conversion goes through float). A null norm
// weight skips the normalization of that input (rope_apply alone); a null k processes q only. Pair p of a head is
// on the time axis for p < 22, height for p < 43, width otherwise; the token's position is
// (start_frame + m / (h w), (m / w) % h, m % w) and (c, s) = freq[0/1][position][p] (table [2, P, 64]).
// Rows m >= f h w (padding) are normalized but not rotated. Outputs are bf16 [M, H*D] (row stride ldo).
//
// quant_q: Sage's per-thread int8 Q (kernels/sage_kv.py:112-124): per 32-token block and head, lane l = 0..7 owns
// tokens l, l+8, l+16, l+24 with scale = max|x| / 127 + 1e-7, q = trunc(x / scale +- 0.5).
#include "wdl_common.h"

namespace {

using namespace wdl;

constexpr int MAXCH = 8;

// four consecutive table entries (16 bytes for fp32, 32 for fp64; p0 is a multiple of 4, so both are aligned)
__device__ __forceinline__ void load4(const float* p, float (&v)[4]) {
    const float4 r = *reinterpret_cast<const float4*>(p);
    v[0] = r.x, v[1] = r.y, v[2] = r.z, v[3] = r.w;
}
__device__ __forceinline__ void load4(const double* p, double (&v)[4]) {
    const double2 r0 = reinterpret_cast<const double2*>(p)[0], r1 = reinterpret_cast<const double2*>(p)[1];
    v[0] = r0.x, v[1] = r0.y, v[2] = r1.x, v[3] = r1.y;
}

struct NormRopeArgs {
    const uint16_t* q;
    int64_t ldq;
    const uint16_t* k;
    int64_t ldk;
    const uint16_t* wq;  // bf16 [H*D]
    const uint16_t* wk;
    const void* freq;    // [2, P, D/2] fp32 or fp64
    int64_t P;
    int64_t M, C;        // rows, columns (H * D)
    int f, h, w, start;
    float eps;
    uint16_t* qo;
    uint16_t* ko;
    int64_t ldo;
    int items;           // inputs per row: 2 (q and k) or 1 (q only)
    int vec;             // the table is 16-byte aligned: 4 entries per vector load
};

__device__ __forceinline__ void load8(const uint16_t* p, float* f) {
    uint4 raw = *reinterpret_cast<const uint4*>(p);
    const uint32_t wv[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = __uint_as_float(wv[j] << 16);
        f[2 * j + 1] = __uint_as_float(wv[j] & 0xffff0000u);
    }
}

// Two waves per (row, q|k), two rows per workgroup. Lane l of the row's first wave owns the chunks c = l + 64 i
// for i < I0 = ceil(I / 2) (I = ceil(chunks / 64)), of the second wave those for I0 <= i < I: the same lane->chunk
// map as one wave over the row. The sum of squares keeps the one-wave order exactly: the first wave's lane sums go
// through LDS and the second wave continues each from there, value by value, then reduces across lanes. Every load
// of a wave (its x chunks, norm weights and rotation table entries) is issued before any arithmetic.
template <typename T>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(NormRopeArgs a) {
    constexpr int CW = MAXCH / 2;  // chunks per lane and wave
    __shared__ float part[2][64];  // the first wave's lane sums, per row slot
    __shared__ float srstd[2];
    // the wave index through readfirstlane: the row, its pointers and the branches on them are then wave-uniform
    // (scalar registers and branches) instead of per-lane values
    const int lane = threadIdx.x % 64, wv = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), slot = wv / 2,
              hw = wv % 2;
    const int64_t item = int64_t(blockIdx.x) * 2 + slot;  // (row, which)
    const bool valid = item < a.items * a.M;
    const int64_t row = valid ? item / a.items : 0;
    const int which = int(item % a.items);
    const uint16_t* src = (which == 0 ? a.q : a.k) + row * (which == 0 ? a.ldq : a.ldk);
    const uint16_t* wt = which == 0 ? a.wq : a.wk;
    uint16_t* dst = (which == 0 ? a.qo : a.ko) + row * a.ldo;
    const T* freq = static_cast<const T*>(a.freq);
    const int64_t chunks = a.C / 8;
    const int nI = int((chunks + 63) / 64), nI0 = (nI + 1) / 2;
    const int i0 = hw == 0 ? 0 : nI0, i1 = hw == 0 ? nI0 : nI;  // this wave's chunk slots [i0, i1)
    const int64_t hwn = int64_t(a.h) * a.w;
    const bool rot = row < int64_t(a.f) * hwn;
    const int pos_t = a.start + int(row / hwn);
    const int pos_h = int((row / a.w) % a.h);
    const int pos_w = int(row % a.w);
    constexpr int half = 64, tpairs = half - 2 * (half / 3), spairs = half / 3;  // 22, 21
    uint4 xr[CW], wr[CW];
    T cs[CW][4], sn[CW][4];
#pragma unroll
    for (int k = 0; k < CW; ++k) {
        const int64_t c = lane + 64 * int64_t(i0 + k);
        xr[k] = wr[k] = make_uint4(0, 0, 0, 0);
        if (valid && i0 + k < i1 && c < chunks) {
            xr[k] = *reinterpret_cast<const uint4*>(src + c * 8);
            if (wt) wr[k] = *reinterpret_cast<const uint4*>(wt + c * 8);
            if (rot) {
                // the chunk's 4 pairs p0 .. p0 + 3: one vector load each of cos and sin when they share an axis
                // (all but the two groups that straddle an axis boundary)
                const int p0 = int((c * 8) % 128) / 2;
                const int ax0 = p0 < tpairs ? 0 : (p0 < tpairs + spairs ? 1 : 2);
                const int ax3 = p0 + 3 < tpairs ? 0 : (p0 + 3 < tpairs + spairs ? 1 : 2);
                if (a.vec && ax0 == ax3) {
                    const int pos = ax0 == 0 ? pos_t : (ax0 == 1 ? pos_h : pos_w);
                    load4(freq + int64_t(pos) * half + p0, cs[k]);
                    load4(freq + (a.P + pos) * half + p0, sn[k]);
                } else {
#pragma unroll
                    for (int p2 = 0; p2 < 4; ++p2) {
                        const int p = p0 + p2;
                        const int pos = p < tpairs ? pos_t : (p < tpairs + spairs ? pos_h : pos_w);
                        cs[k][p2] = freq[int64_t(pos) * half + p];
                        sn[k][p2] = freq[(a.P + pos) * half + p];
                    }
                }
            }
        }
    }
    // sum of squares in the one-wave order: the first wave sums its slots from 0 (absent chunks would add + 0,
    // exact), the second continues each lane's sum through its own slots
    float s = 0.0f;
    if (wt && hw == 0) {
#pragma unroll
        for (int k = 0; k < CW; ++k) {
            const uint32_t xw[4] = {xr[k].x, xr[k].y, xr[k].z, xr[k].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = __uint_as_float(j % 2 == 0 ? xw[j / 2] << 16 : xw[j / 2] & 0xffff0000u);
                if (i0 + k < i1) s = s + v * v;
            }
        }
    }
    if (hw == 0) part[slot][lane] = s;
    __syncthreads();
    if (hw == 1 && wt) {
        float t = part[slot][lane];
#pragma unroll
        for (int k = 0; k < CW; ++k) {
            const uint32_t xw[4] = {xr[k].x, xr[k].y, xr[k].z, xr[k].w};
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                const float v = __uint_as_float(j % 2 == 0 ? xw[j / 2] << 16 : xw[j / 2] & 0xffff0000u);
                if (i0 + k < i1) t = t + v * v;
            }
        }
        t = group_sum<64>(t);
        if (lane == 0) srstd[slot] = 1.0f / sqrtf(t / float(a.C) + a.eps);
    }
    __syncthreads();
    if (!valid) return;
    const float rstd = wt ? srstd[slot] : 1.0f;
#pragma unroll
    for (int k = 0; k < CW; ++k) {
        const int64_t c = lane + 64 * int64_t(i0 + k);
        if (i0 + k >= i1 || c >= chunks) continue;
        const int64_t col = c * 8;
        const uint32_t xw[4] = {xr[k].x, xr[k].y, xr[k].z, xr[k].w};
        const uint32_t ww[4] = {wr[k].x, wr[k].y, wr[k].z, wr[k].w};
        float y[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float x = __uint_as_float(j % 2 == 0 ? xw[j / 2] << 16 : xw[j / 2] & 0xffff0000u);
            if (wt) {
                const float w = __uint_as_float(j % 2 == 0 ? ww[j / 2] << 16 : ww[j / 2] & 0xffff0000u);
                const float n = bf16_to_f32(f32_to_bf16(x * rstd));
                y[j] = bf16_to_f32(f32_to_bf16(n * w));
            } else {
                y[j] = x;
            }
        }
        uint16_t o[8];
#pragma unroll
        for (int p2 = 0; p2 < 4; ++p2) {
            if (rot) {
                const T x1 = T(y[2 * p2]), x2 = T(y[2 * p2 + 1]);
                o[2 * p2] = f32_to_bf16(float(x1 * cs[k][p2] - x2 * sn[k][p2]));
                o[2 * p2 + 1] = f32_to_bf16(float(x2 * cs[k][p2] + x1 * sn[k][p2]));
            } else {
                o[2 * p2] = f32_to_bf16(y[2 * p2]);
                o[2 * p2 + 1] = f32_to_bf16(y[2 * p2 + 1]);
            }
        }
        *reinterpret_cast<uint4*>(dst + col) =
            make_uint4(o[0] | (uint32_t(o[1]) << 16), o[2] | (uint32_t(o[3]) << 16), o[4] | (uint32_t(o[5]) << 16),
                       o[6] | (uint32_t(o[7]) << 16));
    }
}

// one wave per (32-token block, head); lane = 2 * token_in_block + (d half); values of 64 d per lane
__global__ __launch_bounds__(256) void quant_q_kernel(const uint16_t* x, int64_t ldx, int64_t n, int64_t H,
                                                      int64_t blocks, int8_t* q, float* q_scale) {
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / 64), lane = threadIdx.x % 64;
    const int64_t item = int64_t(blockIdx.x) * 4 + wave;  // (block, head)
    if (item >= blocks * H) return;
    const int64_t blk = item / H, h = item % H;
    const int tok = lane / 2, dh = lane % 2;
    const int64_t token = blk * 32 + tok;
    const bool live = token < n;
    float v[64];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < 8; ++c) {
        float f[8];
        if (live) load8(x + token * ldx + h * 128 + dh * 64 + c * 8, f);
        else
            for (int j = 0; j < 8; ++j) f[j] = 0.0f;
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            v[c * 8 + j] = f[j];
            amax = fmaxf(amax, fabsf(f[j]));
        }
    }
    // group of lane l8 = tok % 8: tokens l8 + 8k -> lanes 2 * l8 + 16 k + dh: xor over lane bits 0, 4, 5
    amax = xor_max<32>(xor_max<16>(xor_max<1>(amax)));
    const float scale = amax / 127.0f + 1e-7f;
    if (lane < 16 && (lane % 2) == 0) q_scale[h * blocks * 8 + blk * 8 + lane / 2] = scale;
    if (!live) return;
    int8_t* dst = q + token * (H * 128) + h * 128 + dh * 64;
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float y = v[c * 16 + b * 4 + e] / scale;
                const float r = __builtin_truncf(y + (y >= 0.0f ? 0.5f : -0.5f));
                word |= (uint32_t(int32_t(r)) & 0xffu) << (8 * e);
            }
            w[b] = word;
        }
        *reinterpret_cast<uint4*>(dst + c * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

}  // namespace

extern "C" int wdl_qk_norm_rope(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* wq,
                                const void* wk, const void* freq, int freq_dtype, int64_t positions, int64_t M,
                                int64_t heads, int f, int h, int w, int start_frame, float eps, void* q_out,
                                void* k_out, int64_t ldo, hipStream_t stream) {
    const int64_t C = heads * 128;
    const int items = k ? 2 : 1;
    if (M < 0 || heads <= 0 || ldq < C || (k && ldk < C) || ldo < C || f < 0 || h <= 0 || w <= 0 || start_frame < 0)
        return fail(WDL_EINVAL, "qk_norm_rope: bad shape");
    if (freq_dtype != WDL_F32 && freq_dtype != WDL_F64) return fail(WDL_EINVAL, "qk_norm_rope: table must be fp32 or fp64");
    if (int64_t(f) * h * w > M) return fail(WDL_EINVAL, "qk_norm_rope: grid exceeds the rows");
    if (start_frame + f > positions || h > positions || w > positions)
        return fail(WDL_EINVAL, "qk_norm_rope: grid or offset exceeds the frequency table");
    if (!q || !freq || !q_out || (k && !k_out)) return fail(WDL_EINVAL, "qk_norm_rope: null pointer");
    if (C > 64 * 8 * MAXCH) return fail(WDL_EINVAL, "qk_norm_rope: rows above 4096 values");
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(q_out) |
         reinterpret_cast<uintptr_t>(k_out) | (ldq * 2) | (k ? ldk * 2 : 0) | (ldo * 2)) % 16)
        return fail(WDL_EINVAL, "qk_norm_rope: rows must be 16-byte aligned");
    if (M == 0) return WDL_OK;
    NormRopeArgs a{static_cast<const uint16_t*>(q), ldq, static_cast<const uint16_t*>(k), ldk,
                   static_cast<const uint16_t*>(wq), static_cast<const uint16_t*>(wk), freq, positions, M, C,
                   f, h, w, start_frame, eps, static_cast<uint16_t*>(q_out), static_cast<uint16_t*>(k_out), ldo,
                   items, reinterpret_cast<uintptr_t>(freq) % 16 == 0};
    const unsigned grid = unsigned((items * M + 1) / 2);
    if (freq_dtype == WDL_F64) qk_norm_rope_kernel<double><<<grid, 256, 0, stream>>>(a);
    else qk_norm_rope_kernel<float><<<grid, 256, 0, stream>>>(a);
    return check_launch("qk_norm_rope");
}

extern "C" int wdl_quant_q(const void* x, int64_t ldx, int64_t n, int64_t heads, void* q, float* q_scale,
                           hipStream_t stream) {
    if (n < 0 || heads <= 0 || ldx < heads * 128) return fail(WDL_EINVAL, "quant_q: bad shape");
    if (!x || !q || !q_scale) return fail(WDL_EINVAL, "quant_q: null pointer");
    if ((reinterpret_cast<uintptr_t>(x) | (ldx * 2)) % 16) return fail(WDL_EINVAL, "quant_q: unaligned rows");
    const int64_t blocks = (n + 127) / 128 * 4;
    if (n == 0) return WDL_OK;
    quant_q_kernel<<<unsigned((blocks * heads + 3) / 4), 256, 0, stream>>>(
        static_cast<const uint16_t*>(x), ldx, n, heads, blocks, static_cast<int8_t*>(q), q_scale);
    return check_launch("quant_q");
}
