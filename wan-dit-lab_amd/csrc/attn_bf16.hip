// bf16 attention on gfx950 matrix cores (fp32 softmax), for the cross-attention over a prompt's keys: the
// computation of torch's scaled_dot_product_attention on bf16 Q, K, V as MultiHeadAttention.forward runs it for
// the context (models/multi_head_attention.py:28-44; generation/causal.py:418-420 keep SDPA for cross-attention).
//
//   s[q][t] = (q . k_t) sm_scale        (bf16 products, fp32 sums)
//   O[q]    = sum_t softmax_t(s)[q][t] v_t
// online over 64-key blocks in log2 units: m = running max, p = 2^(y - m) in fp32, l = sum of the fp32 p, P rounded to
// bf16 for the P V product (as flash attention does), O accumulated in fp32, out = bf16(O / l).
//
// Operands. Q bf16 [n, H, 128] (row stride ldq), read once per tile into registers. K and V are laid out once per
// prompt by wdl_attn_bf16_prep (the prompt's keys do not change between steps):
//   Kp [H][Lpad][128] bf16, the 16-byte chunks of key row t XOR-swizzled by t % 16;
//   Vp [H][128][Lpad] bf16 (V transposed), in each 16-key group the keys ordered [0..3, 8..11, 4..7, 12..15] and
//      the 16-byte chunks of channel row d inside each 64-key block XOR-swizzled by (d / 2) % 8;
// keys >= L are zero. Both swizzles make the 16-byte reads of 16 consecutive rows (one LDS read phase) hit 16
// distinct bank groups, and both layouts make one 64-key block a straight copy into LDS.
//
// Work split: a workgroup of 2 WPG waves takes 32 WPG queries of one head; its two groups of WPG waves take the key
// blocks in halves, each wave 32 queries, and stream K / V blocks through a 2-stage LDS ring per group
// (global_load_lds, 16 bytes per lane, issued by the group's first 4 waves). WPG is 4, or 5 / 6 when that fits
// every (query tile, head) pair into one round of workgroups (1392 queries x 24 heads: 9 tiles of 160 queries,
// 216 workgroups, where 128-query tiles would need 264). Products are computed transposed so that a lane owns one query:
//   S^T = K Q^T   with v_mfma_f32_32x32x16_bf16 (8 per 32 x 32 tile over d = 128);
//   O^T = V^T P^T with v_mfma_f32_32x32x16_bf16 (4 per 16 keys, one per 32 channels);
// the lane's 32 scores of a block (keys 32 j + 8 g + 4 half + e) are the B operand of the P V product in 16-key
// slices, which is why V's keys are reordered inside each 16-key group. The block max needs one exchange with
// lane ^ 32. Group 1 hands (O, m, l) to group 0 through LDS at the end. When the (query tile, head) pairs number
// between one and two times the CU count and no wider tile fits one round, the first T - CUs workgroups run two
// tiles, one per group over all the key blocks, so the launch takes one round. Tiles are dealt so that each XCD runs a contiguous range of them.
#include "wdl_common.h"

namespace {

using namespace wdl;

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

constexpr int D = 128;
constexpr int RING = 2;                        // stages per group
constexpr int BLK_BYTES = 64 * D * 2;          // one 64-key block of K (or of V), bf16
constexpr int GSTAGE = 2 * BLK_BYTES;          // K then V
constexpr int STAGE = 2 * GSTAGE;              // both groups
constexpr int LPB = 2 * BLK_BYTES / (256 * 16);  // 16-byte loads per loading lane per block (K and V): 8

struct Args {
    const uint16_t* q;
    int64_t ldq;
    const uint16_t* kp;   // [H][Lpad][128]
    const uint16_t* vp;   // [H][128][Lpad]
    uint16_t* out;
    int64_t ldo;
    int64_t n, L, Lpad, H, qtiles;
    float scale_log2;     // sm_scale * log2(e)
    int64_t dual;         // workgroups 0 .. dual - 1 run two tiles (one per group)
};

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

template <int WPG>
__global__ __launch_bounds__(128 * WPG) void attn_bf16_kernel(Args a) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[RING * STAGE];
    static_assert(WPG >= 4 && WPG * (64 * 64 + 128) * 4 <= RING * STAGE, "the hand-over fits the ring's LDS");

    const int t = threadIdx.x, lane = t % 64, half = lane / 32, tok = lane % 32;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);
    const int grp = wave / WPG, sub = wave % WPG;
    const bool loader = sub < 4;  // the group's first 4 waves copy its K / V blocks (uniform per wave)
    // workgroup ids go round-robin over the 8 XCDs: each XCD takes a contiguous range of the tiles, so the query
    // tiles of one head (consecutive tiles) read its K / V through one L2 (otherwise every XCD streams every head's
    // K / V from the memory side)
    const int64_t W = gridDim.x;
    const int64_t w = W % 8 == 0 ? (blockIdx.x % 8) * (W / 8) + blockIdx.x / 8 : blockIdx.x;
    const bool dualwg = w < a.dual;
    const int64_t tile = dualwg ? 2 * w + grp : a.dual + w;
    const int64_t h = tile / a.qtiles, qt = tile % a.qtiles;
    const int64_t q = qt * (32 * WPG) + sub * 32 + tok;
    const bool qlive = q < a.n;
    const int nblk = int(a.Lpad / 64), L32 = int(a.L);  // Lpad < 2^23 (checked by the launcher)
    const bool ragged = L32 % 64 != 0;
    // key blocks of this group: all of them (dual), or its half
    const int nb0 = dualwg ? nblk : (nblk + 1) / 2;
    const int first = grp == 0 || dualwg ? 0 : nb0, count = grp == 0 || dualwg ? nb0 : nblk - nb0;
    const int iters = nb0;  // both groups run the same number of ring steps (barriers match)
    const int last = count > 0 ? first + count - 1 : 0;

    // ring loads: the group's 256 lanes copy a block's K (16 KB contiguous) and V (128 rows of 128 bytes, row
    // stride 2 Lpad bytes) as 4 + 4 loads of 16 bytes per lane
    const uint8_t* kbase = reinterpret_cast<const uint8_t*>(a.kp + h * a.Lpad * D);
    const uint8_t* vbase = reinterpret_cast<const uint8_t*>(a.vp + h * D * a.Lpad);
    const int gl = sub * 64 + lane;  // lane within the group
    uint32_t voff[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        const int slot = j * 256 + gl;  // 16-byte slot of the V block: row slot / 8, chunk slot % 8
        voff[j] = uint32_t((slot / 8) * (2 * a.Lpad) + (slot % 8) * 16);
    }
    auto load_block = [&](int st, int blk) {
        if (!loader) return;
        uint8_t* base = smem + st * STAGE + grp * GSTAGE;
        const uint8_t* kb = kbase + int64_t(blk) * BLK_BYTES;
        const uint8_t* vb = vbase + int64_t(blk) * 128;  // 64 keys x 2 bytes into each channel row
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16s(kb, uint32_t((j * 256 + gl) * 16), lds_addr(base + j * 4096 + sub * 1024));
#pragma unroll
        for (int j = 0; j < 4; ++j) dma16s(vb, voff[j], lds_addr(base + BLK_BYTES + j * 4096 + sub * 1024));
    };
    auto issue = [&](int st, int i) { load_block(st, first + i < last ? first + i : last); };

    // the prologue's loads first, then Q (both in flight together)
    issue(0, 0);
    issue(1, 1);
    bf16x8 qf[8];  // B operand of S^T: query tok, d = 16 s + 8 half .. + 7
#pragma unroll
    for (int s = 0; s < 8; ++s) {
        uint4 r = make_uint4(0u, 0u, 0u, 0u);
        if (qlive) r = *reinterpret_cast<const uint4*>(a.q + q * a.ldq + h * D + 16 * s + 8 * half);
        qf[s] = __builtin_bit_cast(bf16x8, r);
    }

    f32x16 o[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) o[i] = f32x16{};
    float m = -INFINITY, l = 0.0f;
    const int ksw = tok & 15, vsw = (tok >> 1) & 7;  // the read rows' swizzles (rows 32 j + tok, 32 ds + tok)

    // mask: the final block of a ragged L (keys >= L get p = 0); a uniform branch
    auto compute = [&](int st, int blk, bool mask) {
        const uint8_t* K = smem + st * STAGE + grp * GSTAGE;
        const uint8_t* V = K + BLK_BYTES;
        f32x16 s[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const uint8_t* row = K + (32 * j + tok) * 256;
            s[j] = f32x16{};
#pragma unroll
            for (int c = 0; c < 8; ++c) {
                const bf16x8 kf = *reinterpret_cast<const bf16x8*>(row + (((2 * c + half) ^ ksw) * 16));
                s[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[c], s[j], 0, 0, 0);
            }
        }
        // keys of register r of tile j: 64 blk + 32 j + 8 (r / 4) + 4 half + r % 4
        if (mask) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r)
                    if (64 * blk + 32 * j + 8 * (r / 4) + 4 * half + r % 4 >= L32) s[j][r] = -INFINITY;
        }
        // the maximum of the raw scores (scale > 0), then y - m = s * scale - m as one fma per score
        float mx = -INFINITY;
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
            for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[j][r]);
        mx = xor_max<32>(mx);  // the other lane half's maximum
        const float mn = fmaxf(m, mx * a.scale_log2);
        const float alpha = __builtin_amdgcn_exp2f(m - mn);  // m = -inf on the first block: 0
        float ls = 0.0f;
        bf16x8 pf[4];  // B operand of O^T per 16-key slice u: keys 16 u + 4 half + e, 16 u + 8 + 4 half + e
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int j = u / 2, g0 = 2 * (u % 2);
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const int r = 4 * (g0 + k / 4) + k % 4;
                // raw v_exp_f32 (results below 2^-126 flush to 0, far below bf16's resolution of P)
                const float p = __builtin_amdgcn_exp2f(fmaf(s[j][r], a.scale_log2, -mn));
                ls = ls + p;
                pf[u][k] = static_cast<__bf16>(p);
            }
        }
        l = l * alpha + ls;
        m = mn;
        if (__any(alpha != 1.0f)) {
#pragma unroll
            for (int ds = 0; ds < 4; ++ds)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[ds][e] *= alpha;
        }
#pragma unroll
        for (int ds = 0; ds < 4; ++ds) {
            const uint8_t* row = V + (32 * ds + tok) * 128;
#pragma unroll
            for (int u = 0; u < 4; ++u) {
                const bf16x8 vf = *reinterpret_cast<const bf16x8*>(row + (((2 * u + half) ^ vsw) * 16));
                o[ds] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[u], o[ds], 0, 0, 0);
            }
        }
    };

    for (int i = 0; i < iters; ++i) {
        const int st = i % RING;
        if (i + 1 < iters) wait_vmcnt<LPB>();  // block i landed (block i + 1 may still be in flight)
        else wait_vmcnt<0>();
        __syncthreads();
        if (i < count) compute(st, first + i, ragged && first + i == nblk - 1);
        __syncthreads();  // every wave is done reading stage st before it is refilled
        if (i + RING < iters) issue(st, i + RING);
    }
    wait_vmcnt<0>();

    // group 1 hands (O, m, l) to group 0 through the ring's LDS; group 0 merges and writes
    float* xo = reinterpret_cast<float*>(smem) + sub * (64 * 64 + 128);
    if (grp == 1 && !dualwg) {
#pragma unroll
        for (int ds = 0; ds < 4; ++ds)
#pragma unroll
            for (int e = 0; e < 16; ++e) xo[(ds * 16 + e) * 64 + lane] = o[ds][e];
        xo[64 * 64 + lane] = m;
        xo[64 * 64 + 64 + lane] = l;
    }
    __syncthreads();
    if (grp == 1 && !dualwg) return;
    if (!dualwg) {
        const float m1 = xo[64 * 64 + lane], l1 = xo[64 * 64 + 64 + lane];
        const float mt = fmaxf(m, m1);
        const float a0 = __builtin_amdgcn_exp2f(m - mt), a1 = __builtin_amdgcn_exp2f(m1 - mt);
        l = l * a0 + l1 * a1;
#pragma unroll
        for (int ds = 0; ds < 4; ++ds)
#pragma unroll
            for (int e = 0; e < 16; ++e) o[ds][e] = o[ds][e] * a0 + xo[(ds * 16 + e) * 64 + lane] * a1;
    }
    const float lt = xor_sum<32>(l);  // the two lane halves summed different keys
    const float inv = 1.0f / lt;
    // The wave's 32 x 128 bf16 outputs go through its own LDS area (the hand-over slot it has just read, or for a
    // dual workgroup a slot per wave), rows of 272 bytes, and leave as whole 256-byte query rows: 16 bytes per lane,
    // four rows per store instead of 32 rows in 8-byte pieces.
    constexpr int SROW = 136;  // staged row, in bf16 elements (128 + 8 pad)
    static_assert(32 * SROW * 2 <= (64 * 64 + 128) * 4 && 2 * WPG * 32 * SROW * 2 <= RING * STAGE, "staging fits");
    uint16_t* stg = dualwg ? reinterpret_cast<uint16_t*>(smem) + (grp * WPG + sub) * 32 * SROW
                           : reinterpret_cast<uint16_t*>(xo);
#pragma unroll
    for (int ds = 0; ds < 4; ++ds)
#pragma unroll
        for (int g = 0; g < 4; ++g) {
            const int d = 32 * ds + 8 * g + 4 * half;
            uint16_t r[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) r[e] = f32_to_bf16(o[ds][4 * g + e] * inv);
            *reinterpret_cast<uint2*>(stg + tok * SROW + d) =
                make_uint2(r[0] | (uint32_t(r[1]) << 16), r[2] | (uint32_t(r[3]) << 16));
        }
    const int64_t q0 = qt * (32 * WPG) + sub * 32;  // the wave's first query
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = 4 * i + lane / 16, c = lane % 16;
        const uint4 v = *reinterpret_cast<const uint4*>(stg + row * SROW + 8 * c);
        if (q0 + row < a.n) *reinterpret_cast<uint4*>(a.out + (q0 + row) * a.ldo + h * D + 8 * c) = v;
    }
}

// K, V bf16 [L, H, 128] (token strides ldk, ldv) -> Kp, Vp (layouts above). One thread per 16-byte chunk of Kp and
// one per 16-byte chunk of Vp; keys >= L are zero.
__global__ __launch_bounds__(256) void attn_bf16_prep_kernel(const uint16_t* k, int64_t ldk, const uint16_t* v,
                                                             int64_t ldv, int64_t L, int64_t Lpad, int64_t H,
                                                             uint16_t* kp, uint16_t* vp) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    const int64_t kchunks = H * Lpad * 16;
    if (i < kchunks) {
        // physical chunk pc of key row (h, t) holds logical chunk pc ^ (t % 16): d = 8 (pc ^ (t % 16)) .. + 7
        const int64_t hh = i / (Lpad * 16), t = (i / 16) % Lpad;
        const int pc = int(i % 16), c = pc ^ int(t % 16);
        uint4 r = make_uint4(0u, 0u, 0u, 0u);
        if (t < L) r = *reinterpret_cast<const uint4*>(k + t * ldk + hh * D + 8 * c);
        *reinterpret_cast<uint4*>(kp + i * 8) = r;
        return;
    }
    const int64_t j = i - kchunks;
    if (j >= H * D * (Lpad / 8)) return;
    // Vp chunk: head hh, channel d, block b, physical chunk pc -> logical chunk c = pc ^ ((d / 2) % 8): keys of the
    // 16-key group u = c / 2 in positions 8 (c % 2) .. + 7, i.e. keys 16 u + 4 (c % 2) + {0..3} and + 8 + {0..3}
    const int64_t hh = j / (D * (Lpad / 8)), d = (j / (Lpad / 8)) % D, cb = j % (Lpad / 8);
    const int64_t b = cb / 8;
    const int pc = int(cb % 8), c = pc ^ int((d / 2) % 8);
    const int64_t t0 = 64 * b + 16 * (c / 2) + 4 * (c % 2);
    uint16_t r[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        const int64_t tt = t0 + (e < 4 ? e : 8 + e - 4);
        r[e] = tt < L ? v[tt * ldv + hh * D + d] : uint16_t(0);
    }
    *reinterpret_cast<uint4*>(vp + (hh * D + d) * Lpad + 8 * cb) =
        make_uint4(r[0] | (uint32_t(r[1]) << 16), r[2] | (uint32_t(r[3]) << 16), r[4] | (uint32_t(r[5]) << 16),
                   r[6] | (uint32_t(r[7]) << 16));
}

}  // namespace

extern "C" int64_t wdl_attn_bf16_prep_elems(int64_t L, int64_t heads) {
    if (L < 1 || heads <= 0) return 0;
    return heads * ((L + 63) / 64 * 64) * D;
}

extern "C" int wdl_attn_bf16_prep(const void* k, int64_t ldk, const void* v, int64_t ldv, int64_t L, int64_t heads,
                                  void* kp, void* vp, hipStream_t stream) {
    if (L < 1 || heads <= 0 || ldk < heads * D || ldv < heads * D)
        return fail(WDL_EINVAL, "attn_bf16_prep: bad shape L=%lld heads=%lld", (long long)L, (long long)heads);
    if (!k || !v || !kp || !vp) return fail(WDL_EINVAL, "attn_bf16_prep: null pointer");
    if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(kp) | reinterpret_cast<uintptr_t>(vp) |
         (ldk * 2)) % 16 || reinterpret_cast<uintptr_t>(v) % 2)
        return fail(WDL_EINVAL, "attn_bf16_prep: K rows, Kp and Vp must be 16-byte aligned");
    const int64_t Lpad = (L + 63) / 64 * 64;
    const int64_t chunks = heads * Lpad * 16 + heads * D * (Lpad / 8);
    attn_bf16_prep_kernel<<<unsigned((chunks + 255) / 256), 256, 0, stream>>>(
        static_cast<const uint16_t*>(k), ldk, static_cast<const uint16_t*>(v), ldv, L, Lpad, heads,
        static_cast<uint16_t*>(kp), static_cast<uint16_t*>(vp));
    return check_launch("attn_bf16_prep");
}

extern "C" int wdl_attn_bf16(const void* q, int64_t ldq, const void* kp, const void* vp, int64_t n, int64_t L,
                             int64_t heads, float sm_scale, void* out, int64_t ldo, hipStream_t stream) {
    if (n < 0 || L < 1 || heads <= 0 || ldq < heads * D || ldo < heads * D)
        return fail(WDL_EINVAL, "attn_bf16: bad shape n=%lld L=%lld heads=%lld", (long long)n, (long long)L,
                    (long long)heads);
    if (!q || !kp || !vp || !out) return fail(WDL_EINVAL, "attn_bf16: null pointer");
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) | reinterpret_cast<uintptr_t>(kp) |
         reinterpret_cast<uintptr_t>(vp) | (ldq * 2) | (ldo * 2)) % 16)
        return fail(WDL_EINVAL, "attn_bf16: Q / out rows, Kp and Vp must be 16-byte aligned");
    const int64_t Lpad = (L + 63) / 64 * 64;
    if (2 * Lpad * 128 >= (int64_t(1) << 31)) return fail(WDL_EINVAL, "attn_bf16: L=%lld too long", (long long)L);
    if (n == 0) return WDL_OK;
    // the narrowest query tile (32 WPG queries) whose (tile, head) pairs fit one round of workgroups; else 128
    const int64_t cus = cu_count();
    int wpg = 4;
    for (int w = 4; w <= 6; ++w)
        if (cus > 0 && (n + 32 * w - 1) / (32 * w) * heads <= cus) {
            wpg = w;
            break;
        }
    const int64_t qtiles = (n + 32 * wpg - 1) / (32 * wpg), T = qtiles * heads;
    const int64_t dual = cus > 0 && T > cus && T <= 2 * cus ? T - cus : 0;
    const int64_t W = T - dual;
    Args a{static_cast<const uint16_t*>(q), ldq, static_cast<const uint16_t*>(kp), static_cast<const uint16_t*>(vp),
           static_cast<uint16_t*>(out), ldo, n, L, Lpad, heads, qtiles, sm_scale * 1.4426950408889634f, dual};
    if (wpg == 5) attn_bf16_kernel<5><<<unsigned(W), 640, 0, stream>>>(a);
    else if (wpg == 6) attn_bf16_kernel<6><<<unsigned(W), 768, 0, stream>>>(a);
    else attn_bf16_kernel<4><<<unsigned(W), 512, 0, stream>>>(a);
    return check_launch("attn_bf16");
}
