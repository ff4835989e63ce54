// Sage-2 style attention on gfx950: int8 Q K^T, fp32 online softmax, fp8 P V, non-causal over L keys
// (the computation of live::sage_sm89, native/ops/sage_ops.cpp:12-19, on this build's operand layouts).
//
//   s[q][t]  = q_scale[q] * k_scale[t] * (q_i8 . k_i8)               (exact int32 dot product, then fp32)
//   O[q][d]  = sum_t softmax_t(s * sm_scale)[q][t] * v_fp8[t][d] * v_scale[d]
// P is rounded to e4m3 after scaling by 448 (its full range), the PV products accumulate in fp32 and the row sum
// uses the unrounded P.
//
// Work split: one workgroup = 128 queries of one head (4 waves x 32 queries); key blocks of 64 are staged in LDS
// (double buffered through registers) and shared by the 4 waves. Both products are computed transposed:
//   S^T = K Q^T with v_mfma_i32_32x32x32_i8 (4 per 32x32 tile over d = 128), and
//   O^T = V^T P^T with v_mfma_f32_32x32x64_f8f6f4 (one per 32 channels per 64-key block),
// so a lane owns one query (lane % 32) throughout: its row max and sum need one exchange with lane ^ 32, the
// rescale of O by exp(m_old - m_new) is lane-uniform, and its 32 probabilities of a 64-key block are exactly the
// B operand of the PV product in the V order written by wdl_sage_prep.
// Layouts: q_i8 [n, H, 128] (row stride ldq) with q_scale [H, ceil(n/128)*32] (Sage's per-thread groups);
// k_i8 [H, Lpad, 128] with k_scale [H, Lpad/16]; v_fp8 [H, 128, Lpad]; v_scale [H, 128]; out bf16 [n, H, 128]
// (row stride ldo).
#include "wdl_common.h"

namespace {

using namespace wdl;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int D = 128;
constexpr int KSTRIDE = 144;  // LDS row stride of the K tile (bytes)
constexpr int VSTRIDE = 80;   // LDS row stride of the V tile (bytes)

struct AttnArgs {
    const int8_t* q;
    int64_t ldq;
    const float* q_scale;
    const int8_t* k;
    const float* k_scale;
    const uint8_t* v;
    const float* v_scale;
    uint16_t* out;
    int64_t ldo;
    int64_t n, L, Lpad, H;
    float sm_scale_log2;  // sm_scale * log2(e)
};

__global__ __launch_bounds__(256) void sage_attn_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(16))) uint8_t sK[2][64 * KSTRIDE];
    __shared__ __attribute__((aligned(16))) uint8_t sV[2][D * VSTRIDE];
    __shared__ float sKs[2][4];

    const int t = threadIdx.x, lane = t % 64, wave = t / 64, half = lane / 32;
    const int64_t h = blockIdx.y;
    const int64_t q = int64_t(blockIdx.x) * 128 + wave * 32 + lane % 32;
    const bool qlive = q < a.n;
    const int64_t qblocks8 = (a.n + 127) / 128 * 32;

    // Q fragment: B operand of S^T = K Q^T, chunk c covers d = 32c .. 32c + 31, lane half -> 16 of them
    i32x4 qf[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        if (qlive) {
            const uint4 r = *reinterpret_cast<const uint4*>(a.q + q * a.ldq + h * D + 32 * c + 16 * half);
            qf[c] = i32x4{int(r.x), int(r.y), int(r.z), int(r.w)};
        } else {
            qf[c] = i32x4{0, 0, 0, 0};
        }
    }
    const float qs = qlive ? a.q_scale[h * qblocks8 + (q / 32) * 8 + q % 8] : 0.0f;
    const float cq = qs * a.sm_scale_log2;

    const int64_t nblk = a.Lpad / 64;
    const int8_t* kbase = a.k + h * a.Lpad * D;
    const uint8_t* vbase = a.v + h * D * a.Lpad;
    uint4 kreg[2], vreg[2];
    float ksreg = 0.0f;
    auto fetch = [&](int64_t b) {
        // K tile: row t/4, 32 bytes at (t%4)*32; V tile: channel t/2, 32 bytes at (t%2)*32
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            kreg[c] = *reinterpret_cast<const uint4*>(kbase + (b * 64 + t / 4) * D + (t % 4) * 32 + c * 16);
            vreg[c] = *reinterpret_cast<const uint4*>(vbase + int64_t(t / 2) * a.Lpad + b * 64 + (t % 2) * 32 + c * 16);
        }
        if (t < 4) ksreg = a.k_scale[h * (a.Lpad / 16) + b * 4 + t];
    };
    auto stash = [&](int st) {
#pragma unroll
        for (int c = 0; c < 2; ++c) {
            *reinterpret_cast<uint4*>(&sK[st][(t / 4) * KSTRIDE + (t % 4) * 32 + c * 16]) = kreg[c];
            *reinterpret_cast<uint4*>(&sV[st][(t / 2) * VSTRIDE + (t % 2) * 32 + c * 16]) = vreg[c];
        }
        if (t < 4) sKs[st][t] = ksreg;
    };

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x16{};
    float m = -INFINITY, l = 0.0f;
    const i32x16 izero = {};
    const f32x16 fzero = {};

    fetch(0);
    stash(0);
    for (int64_t b = 0; b < nblk; ++b) {
        const int st = int(b & 1);
        __syncthreads();
        if (b + 1 < nblk) fetch(b + 1);
        // S^T for the two 32-key tiles of the block
        float s[32];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            i32x16 acc = izero;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint4 r = *reinterpret_cast<const uint4*>(&sK[st][(32 * j + lane % 32) * KSTRIDE + 32 * c + 16 * half]);
                const i32x4 kf = {int(r.x), int(r.y), int(r.z), int(r.w)};
                acc = __builtin_amdgcn_mfma_i32_32x32x32_i8(kf, qf[c], acc, 0, 0, 0);
            }
            // key of register r: 32j + 8(r/4) + 4*half + r%4; its scale group (t % 8) / 2 = 2*half + (r%4)/2
            const float ks0 = sKs[st][2 * half], ks1 = sKs[st][2 * half + 1];
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int64_t key = b * 64 + 32 * j + 8 * (r / 4) + 4 * half + r % 4;
                const float v = float(acc[r]) * ((r % 4) < 2 ? ks0 : ks1);
                s[16 * j + r] = key < a.L ? v : -INFINITY;
            }
        }
        float mb = s[0];
#pragma unroll
        for (int r = 1; r < 32; ++r) mb = fmaxf(mb, s[r]);
        mb = fmaxf(mb, __shfl_xor(mb, 32));
        const float mn = fmaxf(m, mb);
        const float alpha = exp2f((m - mn) * cq);
        const float bias = -mn * cq;
        float ls = 0.0f;
        uint32_t pw[8];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            float p[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                p[e] = exp2f(fmaf(s[4 * w + e], cq, bias));
                ls = ls + p[e];
            }
            uint32_t word = __builtin_amdgcn_cvt_pk_fp8_f32(p[0] * 448.0f, p[1] * 448.0f, 0, false);
            word = __builtin_amdgcn_cvt_pk_fp8_f32(p[2] * 448.0f, p[3] * 448.0f, word, true);
            pw[w] = word;
        }
        l = l * alpha + ls;
        m = mn;
        const i32x8 pf = {int(pw[0]), int(pw[1]), int(pw[2]), int(pw[3]), int(pw[4]), int(pw[5]), int(pw[6]), int(pw[7])};
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) {
            const uint8_t* src = &sV[st][(32 * ds + lane % 32) * VSTRIDE + 32 * half];
            const uint4 v0 = *reinterpret_cast<const uint4*>(src), v1 = *reinterpret_cast<const uint4*>(src + 16);
            const i32x8 vf = {int(v0.x), int(v0.y), int(v0.z), int(v0.w), int(v1.x), int(v1.y), int(v1.z), int(v1.w)};
#pragma unroll
            for (int e = 0; e < 16; ++e) o[ds][e] *= alpha;
            o[ds] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf, o[ds], 0, 0, 0, 0, 0, 0);
        }
        if (b + 1 < nblk) stash(st ^ 1);
    }
    const float lt = l + __shfl_xor(l, 32);
    if (!qlive) return;
    const float inv = 1.0f / (lt * 448.0f);
    uint16_t* dst = a.out + q * a.ldo + h * D;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * ds + 8 * g + 4 * half;
            uint16_t r[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = f32_to_bf16(o[ds][4 * g + e] * inv * a.v_scale[h * D + d + e]);
            *reinterpret_cast<uint2*>(dst + d) = make_uint2(r[0] | (uint32_t(r[1]) << 16), r[2] | (uint32_t(r[3]) << 16));
        }
    }
}

}  // namespace

extern "C" int wdl_sage_attn(const void* q_i8, int64_t ldq, const float* q_scale, const void* k_i8,
                             const float* k_scale, const void* v_fp8, const float* v_scale, int64_t n, int64_t L,
                             int64_t heads, float sm_scale, void* out, int64_t ldo, hipStream_t stream) {
    if (n < 0 || L < 1 || heads <= 0 || ldq < heads * D || ldo < heads * D)
        return fail(WDL_EINVAL, "sage_attn: bad shape n=%lld L=%lld", (long long)n, (long long)L);
    if (!q_i8 || !q_scale || !k_i8 || !k_scale || !v_fp8 || !v_scale || !out)
        return fail(WDL_EINVAL, "sage_attn: null pointer");
    if ((reinterpret_cast<uintptr_t>(q_i8) | reinterpret_cast<uintptr_t>(out) | ldq | (ldo * 2)) % 16)
        return fail(WDL_EINVAL, "sage_attn: unaligned rows");
    if (n == 0) return WDL_OK;
    const int64_t Lpad = (L + 63) / 64 * 64;
    AttnArgs a{static_cast<const int8_t*>(q_i8), ldq, q_scale, static_cast<const int8_t*>(k_i8), k_scale,
               static_cast<const uint8_t*>(v_fp8), v_scale, static_cast<uint16_t*>(out), ldo, n, L, Lpad, heads,
               sm_scale * 1.4426950408889634f};
    sage_attn_kernel<<<dim3(unsigned((n + 127) / 128), unsigned(heads)), 256, 0, stream>>>(a);
    return check_launch("sage_attn");
}
