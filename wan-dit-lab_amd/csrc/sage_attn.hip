// Sage-2 style attention on gfx950: int8 Q K^T, fp32 online softmax, fp8 P V, non-causal over L keys
// (the computation of live::sage_sm89, native/ops/sage_ops.cpp:12-19, on this build's operand layouts).
//
//   s[q][t]  = q_scale[q] * k_scale[t] * (q_i8 . k_i8)               (exact int32 dot product, then fp32)
//   O[q][d]  = sum_t softmax_t(s * sm_scale)[q][t] * v_fp8[t][d] * v_scale[d]
// In log2 units y = s * sm_scale * log2(e); per 64-key block P448 = 2^(y - m + log2 448) (the e4m3 range folded into
// the exponent: P448 <= 448) is rounded to e4m3 for the PV product, accumulated in fp32; the row sum l uses the
// unrounded P448 and the output is O / l * v_scale.
//
// Work split: one workgroup = 128 queries of one head and 8 waves: two groups of 4 waves split the key blocks in
// halves (so every SIMD runs two waves), each wave owning 32 queries. A group streams its 64-key blocks of K
// (int8 [64][128]) and V (fp8 [128][64], this build's token order) straight from global memory into a 4-stage LDS
// ring (global_load_lds, 16 bytes per lane, 4 loads per wave per block, issued 3 blocks ahead, waited for with an
// explicit vmcnt); rows are 64 bytes with their 16-byte quarters XOR-swizzled by (row / 4) % 4. Both groups step
// through the same number of ring steps (the shorter one idles through its last), so the barriers match.
// Both products are computed transposed:
//   S^T = K Q^T with v_mfma_i32_32x32x32_i8 (4 per 32x32 tile over d = 128), and
//   O^T = V^T P^T with v_mfma_f32_32x32x64_f8f6f4 (one per 32 channels per 64-key block),
// so a lane owns one query (lane % 32) throughout: the block max needs one exchange with lane ^ 32, and its 32
// probabilities of a block are exactly the B operand of the PV product. Per score the vector work is an integer
// max, a conversion, one fma, one exp2, one add and half a pack; the rescale of O by 2^(m_old - m_new) is skipped
// when no lane's max moved, and key masking runs only in the final partial block. At the end the second group
// hands (O, m, l) over through LDS and the first merges and writes.
// Layouts: q_i8 [n, H, 128] (row stride ldq) with q_scale [H, ceil(n/128)*32] (Sage's per-thread groups);
// k_i8 [H, Lpad, 128] with k_scale [H, Lpad/16]; v_fp8 [H, 128, Lpad]; v_scale [H, 128]; out bf16 [n, H, 128]
// (row stride ldo).
#include "wdl_common.h"

#include <type_traits>

namespace {

using namespace wdl;

typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef int i32x8 __attribute__((ext_vector_type(8)));
typedef int i32x16 __attribute__((ext_vector_type(16)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int D = 128;
constexpr int STAGES = 4;
constexpr int LPB = 4;                    // loads per wave per block: 2 of K, 2 of V
constexpr int KT = 64 * D, VT = D * 64;   // bytes of a K / V block
constexpr int GSTAGE = KT + VT;           // one group's share of a stage
constexpr int STAGE = 2 * GSTAGE;
constexpr int KS_MAX = 2048;              // k scales held in LDS: L <= 32768 keys
constexpr float LOG2_448 = 8.807354922057604f;

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

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// 64 lanes x 16 bytes from per-lane global addresses to LDS [m0, m0 + 1024)
__device__ __forceinline__ void dma16(const void* g, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

__global__ __launch_bounds__(512) void sage_attn_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE];
    __shared__ float sKs[KS_MAX];

    const int t = threadIdx.x, lane = t % 64, half = lane / 32;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);
    const int grp = wave / 4, sub = wave % 4;
    const int64_t h = blockIdx.y;
    const int64_t q = int64_t(blockIdx.x) * 128 + sub * 32 + lane % 32;
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

    const int64_t nks = a.Lpad / 16;
    for (int64_t i = t; i < nks; i += 512) sKs[i] = a.k_scale[h * nks + i];

    // full key blocks of this wave's group: [first, first + count); both groups run `iters` ring steps. A ragged
    // final block (L % 64 != 0) is group 1's, in a masked step after the ring.
    const int64_t nblk = a.Lpad / 64;
    const bool ragged = (a.L % 64) != 0;
    const int64_t nfull = ragged ? nblk - 1 : nblk, nb0 = (nfull + 1) / 2;
    const int64_t first = grp == 0 ? 0 : nb0, count = grp == 0 ? nb0 : nfull - nb0;
    const int64_t last = count > 0 ? first + count - 1 : 0;
    const int64_t iters = nb0;

    // this lane's load slots (block 0); block b adds b * 64 * D bytes of K, b * 64 bytes of V
    const int8_t* kbase = a.k + h * a.Lpad * D;
    const uint8_t* vbase = a.v + h * D * a.Lpad;
    const int8_t* ksrc[2];
    const uint8_t* vsrc[2];
#pragma unroll
    for (int j = 0; j < 2; ++j) {
        const int slot = (sub * 2 + j) * 64 + lane;  // 16-byte slot of the group's 8 KB K or V block
        {
            const int dh = slot / 256, s2 = slot % 256, key = s2 / 4;
            const int lq = (s2 % 4) ^ ((key >> 2) & 3);
            ksrc[j] = kbase + key * D + dh * 64 + lq * 16;
        }
        {
            const int ch = slot / 4, lq = (slot % 4) ^ ((ch >> 2) & 3);
            vsrc[j] = vbase + int64_t(ch) * a.Lpad + lq * 16;
        }
    }
    auto load_block = [&](int st, int64_t b) {  // block b of this group's keys into stage st
        uint8_t* base = smem + st * STAGE + grp * GSTAGE;
#pragma unroll
        for (int j = 0; j < 2; ++j) dma16(ksrc[j] + b * 64 * D, lds_addr(base + (sub * 2 + j) * 1024));
#pragma unroll
        for (int j = 0; j < 2; ++j) dma16(vsrc[j] + b * 64, lds_addr(base + KT + (sub * 2 + j) * 1024));
    };
    auto issue = [&](int st, int64_t i) {  // ring step i's block (clamped to the group's last) into stage st
        const int64_t b = first + i;
        load_block(st, b < last ? b : last);
    };

    // per-lane LDS read offsets: K tile j, chunk c -> (c / 2) * 4096 + (32 j + lane % 32) * 64 + quarter;
    // V channel subtile ds -> KT + (32 ds + lane % 32) * 64 + quarter (two quarters per lane half)
    const int swz = ((lane % 32) >> 2) & 3;
    const int kq[2] = {((0 + half) ^ swz) * 16, ((2 + half) ^ swz) * 16};      // chunk parity 0 / 1
    const int vq0 = ((2 * half) ^ swz) * 16, vq1 = ((2 * half + 1) ^ swz) * 16;
    const int rowoff = (lane % 32) * 64;

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x16{};
    float m = -INFINITY, l = 0.0f;
    const i32x16 izero = {};

    // mask_tag: std::true_type for the final block of a ragged L (keys >= L get P = 0), else std::false_type
    auto compute = [&](int st, int64_t b, auto mask_tag) {
        constexpr bool MASK = decltype(mask_tag)::value;
        const uint8_t* K = smem + st * STAGE + grp * GSTAGE;
        const uint8_t* V = K + KT;
        i32x16 acc[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            acc[j] = izero;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                const uint4 r = *reinterpret_cast<const uint4*>(K + (c / 2) * 4096 + j * 2048 + rowoff + kq[c % 2]);
                acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(i32x4{int(r.x), int(r.y), int(r.z), int(r.w)}, qf[c],
                                                              acc[j], 0, 0, 0);
            }
        }
        // key of register r of tile j: 64 b + 32 j + 8 (r / 4) + 4 half + r % 4; scale group 2 half + (r % 4) / 2
        const float kc0 = sKs[b * 4 + 2 * half] * cq, kc1 = sKs[b * 4 + 2 * half + 1] * cq;
        if (MASK) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (b * 64 + 32 * j + 8 * (r / 4) + 4 * half + r % 4 >= a.L) acc[j][r] = INT32_MIN;
        }
        int mx0 = INT32_MIN, mx1 = INT32_MIN;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                if ((r % 4) < 2) mx0 = max(mx0, acc[j][r]);
                else mx1 = max(mx1, acc[j][r]);
            }
        float mb = fmaxf(float(mx0) * kc0, float(mx1) * kc1);
        mb = fmaxf(mb, __shfl_xor(mb, 32));
        const float mn = fmaxf(m, mb);
        const float alpha = __builtin_amdgcn_exp2f(m - mn);
        const float bias = LOG2_448 - mn;
        float ls = 0.0f;
        uint32_t pw[8];
#pragma unroll
        for (int w = 0; w < 8; ++w) {
            const int j = w / 4;
            float p[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int r = 4 * (w % 4) + e;
                // raw v_exp_f32: results below 2^-126 flush to 0 (below e4m3's range and the sum's precision)
                p[e] = __builtin_amdgcn_exp2f(fmaf(float(acc[j][r]), (r % 4) < 2 ? kc0 : kc1, bias));
                if (MASK && acc[j][r] == INT32_MIN) p[e] = 0.0f;
                ls = ls + p[e];
            }
            uint32_t word = __builtin_amdgcn_cvt_pk_fp8_f32(p[0], p[1], 0, false);
            pw[w] = __builtin_amdgcn_cvt_pk_fp8_f32(p[2], p[3], word, true);
        }
        l = l * alpha + ls;
        m = mn;
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int ds = 0; ds < 4; ++ds)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[ds][e] *= alpha;
        }
        const i32x8 pf = {int(pw[0]), int(pw[1]), int(pw[2]), int(pw[3]), int(pw[4]), int(pw[5]), int(pw[6]), int(pw[7])};
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) {
            const uint8_t* src = V + ds * 2048 + rowoff;
            const uint4 v0 = *reinterpret_cast<const uint4*>(src + vq0), v1 = *reinterpret_cast<const uint4*>(src + vq1);
            const i32x8 vf = {int(v0.x), int(v0.y), int(v0.z), int(v0.w), int(v1.x), int(v1.y), int(v1.z), int(v1.w)};
            o[ds] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf, o[ds], 0, 0, 0, 0, 0, 0);
        }
    };

#pragma unroll
    for (int k = 0; k < STAGES - 1; ++k) issue(k, k);
    for (int64_t i0 = 0; i0 < iters; i0 += STAGES) {
#pragma unroll
        for (int k = 0; k < STAGES; ++k) {
            const int64_t i = i0 + k;
            if (i >= iters) break;
            wait_vmcnt<(STAGES - 2) * LPB>();
            __syncthreads();
            issue((k + STAGES - 1) % STAGES, i + STAGES - 1);
            if (i < count) compute(k, first + i, std::false_type{});
        }
    }
    wait_vmcnt<0>();
    __syncthreads();  // all loads landed and every wave is done with the ring
    if (ragged) {     // the final, partial block: group 1, keys >= L masked
        if (grp == 1) load_block(0, nblk - 1);
        wait_vmcnt<0>();
        __syncthreads();
        if (grp == 1) compute(0, nblk - 1, std::true_type{});
        __syncthreads();  // group 1 is done reading stage 0 before the hand-over overwrites it
    }

    // group 1 hands (O, m, l) to group 0: per sub-wave [64 values][64 lanes] floats, then m and l per lane
    float* xo = reinterpret_cast<float*>(smem) + sub * (64 * 64 + 128);
    if (grp == 1) {
#pragma unroll
        for (int ds = 0; ds < 4; ++ds)
#pragma unroll
            for (int e = 0; e < 16; ++e) xo[(ds * 16 + e) * 64 + lane] = o[ds][e];
        xo[64 * 64 + lane] = m;
        xo[64 * 64 + 64 + lane] = l;
    }
    __syncthreads();
    if (grp == 1) return;
    const float m1 = xo[64 * 64 + lane], l1 = xo[64 * 64 + 64 + lane];
    const float mt = fmaxf(m, m1);
    const float a0 = __builtin_amdgcn_exp2f(m - mt), a1 = __builtin_amdgcn_exp2f(m1 - mt);
    const float lh = l * a0 + l1 * a1;
    const float lt = lh + __shfl_xor(lh, 32);
    if (!qlive) return;
    const float inv = 1.0f / lt;
    uint16_t* dst = a.out + q * a.ldo + h * D;
#pragma unroll
    for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * ds + 8 * g + 4 * half;
            uint16_t r[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float ov = o[ds][4 * g + e] * a0 + xo[(ds * 16 + 4 * g + e) * 64 + lane] * a1;
                r[e] = f32_to_bf16(ov * inv * a.v_scale[h * D + d + e]);
            }
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
    if (Lpad / 16 > KS_MAX) return fail(WDL_EINVAL, "sage_attn: L=%lld above %d keys", (long long)L, KS_MAX * 16);
    if ((reinterpret_cast<uintptr_t>(k_i8) | reinterpret_cast<uintptr_t>(v_fp8)) % 16)
        return fail(WDL_EINVAL, "sage_attn: K / V must be 16-byte aligned");
    AttnArgs a{static_cast<const int8_t*>(q_i8), ldq, q_scale, static_cast<const int8_t*>(k_i8), k_scale,
               static_cast<const uint8_t*>(v_fp8), v_scale, static_cast<uint16_t*>(out), ldo, n, L, Lpad, heads,
               sm_scale * 1.4426950408889634f};
    sage_attn_kernel<<<dim3(unsigned((n + 127) / 128), unsigned(heads)), 512, 0, stream>>>(a);
    return check_launch("sage_attn");
}
