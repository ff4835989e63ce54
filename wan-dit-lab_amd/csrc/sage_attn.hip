// Sage-2 style attention on gfx950: int8 Q K^T, fp32 online softmax, fp8 P V, non-causal over L keys
// (the computation of live::sage_sm89, native/ops/sage_ops.cpp:12-19, on wdl's operand layouts).
//
//   s[q][t]  = q_scale[q] * k_scale[t] * (q_i8 . k_i8)               (exact int32 dot product, then fp32)
//   O[q][d]  = sum_t softmax_t(s * sm_scale)[q][t] * v_fp8[t][d] * v_scale[d]
// In log2 units y = s * sm_scale * log2(e); per 64-key block P448 = 2^(y - m + log2 448 - TAU) is rounded to e4m3
// for the PV product, accumulated in fp32, and the row sum l is the sum of the same rounded values; the output is
// O / l * v_scale. The reference max m is lazy: it moves to the block's max only where that exceeds m by more than
// TAU = 2 (then O and l are rescaled by 2^(m_old - m_new)), so P448 <= 448 always and most blocks rescale nothing.
// (Only the e4m3 underflow threshold moves, by at most TAU bits: values below 2^-9 / 448 of the largest one.)
//
// Work split: one workgroup = 128 queries of one head and 8 waves: two groups of 4 waves split the key blocks in
// halves (so every SIMD runs two waves), each wave owning 32 queries. A group streams its 64-key blocks of K
// (int8 [64][128]) and V (fp8 [128][64], wdl's token order) straight from global memory into a 4-stage LDS
// ring (global_load_lds, 16 bytes per lane, 4 loads per wave per block, issued 3 blocks ahead, waited for with an
// explicit vmcnt); rows are 64 bytes with their 16-byte quarters XOR-swizzled by (row / 4) % 4. Both groups step
// through the same number of ring steps (the shorter one idles through its last), so the barriers match.
// Both products are computed transposed:
//   S^T = K Q^T with v_mfma_i32_32x32x32_i8 (4 per 32x32 tile over d = 128), and
//   O^T = V^T P^T with v_mfma_f32_32x32x64_f8f6f4 (one per 32 channels per 64-key block),
// so a lane owns one query (lane % 32) throughout: the block max needs one exchange with lane ^ 32, and its 32
// probabilities of a block are exactly the B operand of the PV product; l comes from a fifth product of them with
// an all-ones A operand. Per score the vector work is half an integer max (v_max3), one fma (the int32 sum lands
// in an accumulator started at the bits of 1.5 * 2^23, so it is already a float), one exp2 and half a pack; the
// rescale runs only in blocks where some lane's reference max moves. Key masking runs only in the blocks that
// hold keys some query of the tile does not see: a ragged final block (L % 64 != 0), and with the block-causal
// per-frame mode (frame > 0: query q of the chunk, the last n of the L keys, sees the keys before its own frame's
// end) the blocks between the tile's first and last queries' limits. At the end the second group hands (O, m, l)
// over through LDS and the first merges and writes.
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
constexpr float TAU = 2.0f;               // lazy rescale threshold (log2 units)
constexpr int ONES_E4M3 = 0x38383838;     // four e4m3 1.0
constexpr int MAGIC_I = 0x4B400000;       // the bits of MAGIC_F = 1.5 * 2^23
constexpr float MAGIC_F = 12582912.0f;
constexpr int SLOT_FLOATS = 4 * (64 * 64 + 128);  // one partial: per wave [64 values][64 lanes] of O, m, l
constexpr int MAX_WG = 2048;                       // workgroups of a split launch (one per CU)
constexpr int TAIL_DIV = 2;  // the split tiles' key blocks go to the first W / TAIL_DIV workgroups (half as many
                             // pieces to merge, each twice as long: measured 151 -> 148 us at 1392 x 9744, 24 heads)

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
    float* part;          // [2 W][SLOT_FLOATS] partial (O, m, l) of split tiles (null when none is split)
    int64_t W;            // workgroups
    int64_t qtiles;       // query tiles (128 queries) per head
    int64_t D;            // tiles run whole (the first D of the T = qtiles * H); the other T - D are split
    const uint16_t* qb;   // bf16 Q [n, H, 128] (row stride ldq) quantized in the kernel, or null (q, q_scale given)
    int64_t dual;         // workgroups 0 .. dual - 1 run two whole tiles, one per group (D == T; else 0)
    int64_t Wt;           // the first Wt workgroups share the split tiles' key blocks (Wt <= W)
    int64_t frame;        // > 0: block-causal per latent frame of `frame` tokens (query q sees keys below
                          // L - n + (q / frame + 1) frame); 0: every query sees all L keys
};

// Keys [0, limit) that query qq sees.
__device__ __forceinline__ int64_t key_limit(const AttnArgs& a, int64_t qq) {
    if (a.frame <= 0) return a.L;
    const int64_t lim = a.L - a.n + (qq / a.frame + 1) * a.frame;
    return lim < a.L ? lim : a.L;
}

__device__ __forceinline__ uint32_t lds_addr(const void* p) {
    return uint32_t(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// 64 lanes x 16 bytes from a wave-uniform base (scalar registers) plus a 32-bit per-lane offset to LDS
// [m0, m0 + 1024): the address arithmetic of a load stays on the scalar unit
__device__ __forceinline__ void dma16s(const void* base, uint32_t voff, uint32_t lds) {
    asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(base), "{m0}"(lds) : "memory");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    static_assert(N >= 0 && N < 64, "vmcnt range");
    __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// The contributors of a split tile are the workgroups c whose unit range [c U / W, (c + 1) U / W) meets it.
__device__ __forceinline__ int64_t wg_of(int64_t unit, int64_t U, int64_t W) {
    int64_t c = unit * W / U;
    while (c + 1 < W && (c + 1) * U / W <= unit) ++c;
    while (c > 0 && c * U / W > unit) --c;
    return c;
}

__global__ __launch_bounds__(512) void sage_attn_kernel(AttnArgs a) {
    __shared__ __attribute__((aligned(1024))) uint8_t smem[STAGES * STAGE];
    __shared__ float sKs_[2][KS_MAX];  // k scales of each group's head
    __shared__ float sVs_[2][D];       // v_scale of each group's head

    const int t = threadIdx.x, lane = t % 64, half = lane / 32;
    const int wave = __builtin_amdgcn_readfirstlane(t / 64);
    const int grp = wave / 4, sub = wave % 4, tg = t % 256;
    float* sKs = sKs_[grp];
    float* sVs = sVs_[grp];
    const int64_t qblocks8 = (a.n + 127) / 128 * 32;
    const int64_t nblk = a.Lpad / 64, nks = a.Lpad / 16;
    // Work of workgroup w: the whole tiles w, w + W, .. below D (their output written directly), then its share
    // [s0, s1) of the key blocks of the R = T - D remaining tiles, laid end to end (each piece's partial softmax
    // state goes to the workspace slot 2w for its first piece, 2w + 1 for a second; attn_merge_kernel combines them)
    const int64_t w = blockIdx.x;
    // a dual workgroup: its two groups take whole tiles 2w and 2w + 1 with all the key blocks each, no hand-over
    const bool dualwg = w < a.dual;
    const int64_t T = a.qtiles * a.H, R = T - a.D, Usk = R * nblk;
    const int64_t ndp = (a.D - w + a.W - 1) / a.W;
    const int64_t s0 = w < a.Wt ? w * Usk / a.Wt : Usk, s1 = w < a.Wt ? (w + 1) * Usk / a.Wt : Usk;
    int64_t cursor = s0;

    // per-lane LDS read offsets: K tile j, chunk c -> (c / 2) * 4096 + (32 j + lane % 32) * 64 + quarter;
    // V channel subtile ds -> KT + (32 ds + lane % 32) * 64 + quarter (two quarters per lane half)
    const int swz = ((lane % 32) >> 2) & 3;
    const int kq[2] = {((0 + half) ^ swz) * 16, ((2 + half) ^ swz) * 16};      // chunk parity 0 / 1
    const int vq0 = ((2 * half) ^ swz) * 16, vq1 = ((2 * half + 1) ^ swz) * 16;
    const int rowoff = (lane % 32) * 64;
    // the score accumulators start at the bits of 1.5 * 2^23, so the int32 sum s lands in them as the float
    // 1.5 * 2^23 + s (exact for |s| < 2^22; |s| <= 127 * 127 * 128): no int-to-float conversion per score
    const i32x16 imagic = {MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I,
                           MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I, MAGIC_I};
    // group 1's hand-over area (stage 0 of the ring): per sub-wave [64 values][64 lanes] floats, then m and l
    float* xo = reinterpret_cast<float*>(smem) + sub * (64 * 64 + 128);

    int64_t head_loaded = -1;
    for (int64_t seg = 0;; ++seg) {
        // ---- segment: tile `tile` (head h, query tile qt), key blocks [b0, b1)
        int64_t tile, b0, b1, slot = -1;
        if (a.dual > 0) {  // one whole tile per workgroup, or one per group for the first `dual` of them
            if (seg > 0) break;
            tile = dualwg ? 2 * w + grp : a.dual + w;
            b0 = 0, b1 = nblk;
        } else if (seg < ndp) {
            // workgroup ids go round-robin over the 8 XCDs; each XCD takes a contiguous range of the whole tiles, so
            // the query tiles of one head (consecutive tiles) share its K/V in one L2
            const int64_t l = w + seg * a.W;
            tile = a.D % 8 == 0 ? (l % 8) * (a.D / 8) + l / 8 : l;
            b0 = 0, b1 = nblk;
        } else {
            if (cursor >= s1) break;
            b0 = cursor % nblk;
            b1 = b0 + (s1 - cursor) < nblk ? b0 + (s1 - cursor) : nblk;
            tile = a.D + cursor / nblk;
            slot = cursor == s0 ? 2 * w : 2 * w + 1;
            cursor += b1 - b0;
        }
        const int64_t h = tile / a.qtiles, qt = tile % a.qtiles;
        // a new head's k scales: loaded here, written to sKs after the ring prologue and Q are issued (so the load
        // latencies overlap); every wave is past its last read of sKs (segment-end barrier)
        const bool new_head = h != head_loaded;
        float ksr[KS_MAX / 256], vsr = 0.0f;
        if (new_head) {  // each group fills its own copy
#pragma unroll
            for (int i = 0; i < KS_MAX / 256; ++i) {
                const int64_t j = tg + 256 * i;
                ksr[i] = j < nks ? a.k_scale[h * nks + j] : 0.0f;
            }
            if (tg < D) vsr = a.v_scale[h * D + tg];
        }
        const int64_t q = qt * 128 + sub * 32 + lane % 32;
        const bool qlive = q < a.n;

        // Q fragment (B operand of S^T = K Q^T, chunk c covers d = 32c .. 32c + 31, lane half -> 16 of them) and
        // scale, filled after the ring prologue is issued (the Q loads and the first K / V blocks are in flight
        // together)
        i32x4 qf[4];
        float cq;

        // The tile's keys: query q sees keys [0, key_limit(q)); the tile needs blocks [0, nbt) (its last query's
        // limit) and blocks from fet on hold keys some of its queries do not see (its first query's limit; with
        // no frames, only a ragged final block when L % 64 != 0): those run the masked step.
        // (32-bit ring counters: uniform 64-bit compares would run on the vector unit; blocks < 2^9)
        const int64_t qlast = qt * 128 + 127 < a.n ? qt * 128 + 127 : a.n - 1;
        const int nbt = int((key_limit(a, qlast) + 63) / 64), fet = int(key_limit(a, qt * 128) / 64);
        const int64_t lim = key_limit(a, qlive ? q : a.n - 1);  // this lane's query
        // the segment's blocks [b0, bend), split in halves between the groups (both run `iters` ring steps); in a
        // dual workgroup each group runs all the blocks of its own tile and the steps are the longer tile's
        const int ib0 = int(b0), bend = int(b1) < nbt ? int(b1) : nbt, nblocks = bend - ib0;
        int nb0 = (nblocks + 1) / 2, iters = nb0;
        if (dualwg) {
            const int64_t other = 2 * w + 1 - grp, oqt = other % a.qtiles;
            const int64_t olast = oqt * 128 + 127 < a.n ? oqt * 128 + 127 : a.n - 1;
            const int onbt = int((key_limit(a, olast) + 63) / 64);
            nb0 = nblocks;
            iters = nblocks > onbt ? nblocks : onbt;
        }
        const int first = grp == 0 || dualwg ? ib0 : ib0 + nb0, count = grp == 0 || dualwg ? nb0 : nblocks - nb0;
        const int last = count > 0 ? first + count - 1 : ib0;

        // this lane's load offsets inside a block (block b of the head starts at kbase + 64 D b for K, at
        // vbase + 64 b for V: wave-uniform bases)
        const int8_t* kbase = a.k + h * a.Lpad * D;
        const uint8_t* vbase = a.v + h * D * a.Lpad;
        uint32_t koff[2], voff[2];
#pragma unroll
        for (int j = 0; j < 2; ++j) {
            const int slot = (sub * 2 + j) * 64 + lane;  // 16-byte slot of the group's 8 KB K or V block
            {
                const int dh = slot / 256, s2 = slot % 256, key = s2 / 4;
                const int lq = (s2 % 4) ^ ((key >> 2) & 3);
                koff[j] = uint32_t(key * D + dh * 64 + lq * 16);
            }
            {
                const int ch = slot / 4, lq = (slot % 4) ^ ((ch >> 2) & 3);
                voff[j] = uint32_t(ch * a.Lpad + lq * 16);  // 128 Lpad < 2^32 (checked by the launcher)
            }
        }
        auto load_block = [&](int st, int blk) {  // block blk of this group's keys into stage st
            uint8_t* base = smem + st * STAGE + grp * GSTAGE;
            const int8_t* kb = kbase + blk * 64 * D;
            const uint8_t* vb = vbase + blk * 64;
#pragma unroll
            for (int j = 0; j < 2; ++j) dma16s(kb, koff[j], lds_addr(base + (sub * 2 + j) * 1024));
#pragma unroll
            for (int j = 0; j < 2; ++j) dma16s(vb, voff[j], lds_addr(base + KT + (sub * 2 + j) * 1024));
        };
        auto issue = [&](int st, int i) {  // ring step i's block (clamped to the group's last) into stage st
            const int blk = first + i;
            load_block(st, blk < last ? blk : last);
        };

        f32x16 o[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) o[i] = f32x16{};
        // lv: the row sums of the rounded P448 from a fifth PV product against an all-ones A operand (every row of
        // it holds the query's sum, so lv[0] is this lane's l over both lane halves)
        f32x16 lv = {};
        float m = -INFINITY;

        // mask_tag: std::true_type for blocks at or after fet (keys >= the lane's limit get P = 0), else
        // std::false_type
        auto compute = [&](int st, int blk, auto mask_tag) {
            constexpr bool MASK = decltype(mask_tag)::value;
            const uint8_t* K = smem + st * STAGE + grp * GSTAGE;
            const uint8_t* V = K + KT;
            // all eight K fragments are read before the first MFMA, so the reads overlap each other
            uint4 kr[2][4];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    kr[j][c] = *reinterpret_cast<const uint4*>(K + (c / 2) * 4096 + j * 2048 + rowoff + kq[c % 2]);
            i32x16 acc[2];
#pragma unroll
            for (int j = 0; j < 2; ++j) {
                acc[j] = imagic;
#pragma unroll
                for (int c = 0; c < 4; ++c)
                    acc[j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                        i32x4{int(kr[j][c].x), int(kr[j][c].y), int(kr[j][c].z), int(kr[j][c].w)}, qf[c], acc[j], 0, 0, 0);
            }
            __builtin_amdgcn_sched_group_barrier(0x100, 8, 0);  // the eight reads
            __builtin_amdgcn_sched_group_barrier(0x008, 8, 0);  // then the eight MFMAs
            // key of register r of tile j: 64 blk + 32 j + 8 (r / 4) + 4 half + r % 4; scale group 2 half + (r % 4) / 2
            const float kc0 = sKs[blk * 4 + 2 * half] * cq, kc1 = sKs[blk * 4 + 2 * half + 1] * cq;
            if (MASK) {
#pragma unroll
                for (int j = 0; j < 2; ++j)
#pragma unroll
                    for (int r = 0; r < 16; ++r)
                        if (blk * 64 + 32 * j + 8 * (r / 4) + 4 * half + r % 4 >= lim) acc[j][r] = INT32_MIN;
            }
            int mx0 = INT32_MIN, mx1 = INT32_MIN;
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    if ((r % 4) < 2) mx0 = max(mx0, acc[j][r]);
                    else mx1 = max(mx1, acc[j][r]);
                }
            float mb0 = (__int_as_float(mx0) - MAGIC_F) * kc0, mb1 = (__int_as_float(mx1) - MAGIC_F) * kc1;
            if (MASK) {  // a half with every key masked has no maximum (-inf: the reference max does not move)
                mb0 = mx0 == INT32_MIN ? -INFINITY : mb0;
                mb1 = mx1 == INT32_MIN ? -INFINITY : mb1;
            }
            float mb = fmaxf(mb0, mb1);
            {  // the other lane half's block max: v_permlane32_swap (no LDS round trip)
                const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(mb), __float_as_uint(mb), false, false);
                mb = fmaxf(__uint_as_float(sw[0]), __uint_as_float(sw[1]));
            }
            // lazy rescale: the reference max m moves (to the block max) only where the block max exceeds it by
            // more than TAU, so P448 = 2^(y - m + log2 448 - TAU) stays <= 448 and O, l are rescaled in few blocks
            const bool grow = mb > m + TAU;
            if (__any(grow)) {
                const float mn = grow ? mb : m;
                // 1 where m stays (m may still be -inf for a lane that has seen only masked keys: no -inf - -inf)
                const float alpha = grow ? __builtin_amdgcn_exp2f(m - mn) : 1.0f;
#pragma unroll
                for (int ds = 0; ds < 4; ++ds)
#pragma unroll
                    for (int e = 0; e < 16; ++e) o[ds][e] *= alpha;
                lv[0] *= alpha;
                m = mn;
            }
            const float bias = LOG2_448 - TAU - m;
            // y - m + log2 448 - TAU = (1.5 * 2^23 + s) kc + (bias - 1.5 * 2^23 kc): the fma forms the product exactly,
            // so the one extra rounding is the second term's (at most 0.75 kc, a relative 5e-7 kc/ulp of P: far
            // below e4m3's steps)
            const float bias0 = fmaf(-MAGIC_F, kc0, bias), bias1 = fmaf(-MAGIC_F, kc1, bias);
            i32x8 pf;
#pragma unroll
            for (int wd = 0; wd < 8; ++wd) {
                const int j = wd / 4;
                float p[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int r = 4 * (wd % 4) + e;
                    // raw v_exp_f32: results below 2^-126 flush to 0 (below e4m3's range and the sum's precision)
                    p[e] = __builtin_amdgcn_exp2f(fmaf(__int_as_float(acc[j][r]), (r % 4) < 2 ? kc0 : kc1,
                                                       (r % 4) < 2 ? bias0 : bias1));
                    if (MASK && acc[j][r] == INT32_MIN) p[e] = 0.0f;
                }
                // the low pair's conversion keeps the upper half of its old operand, which the high pair's then
                // replaces: any register serves as the old value (p[0]'s bits: no zero to materialise)
                const uint32_t word = __builtin_amdgcn_cvt_pk_fp8_f32(p[0], p[1], __float_as_int(p[0]), false);
                pf[wd] = int(__builtin_amdgcn_cvt_pk_fp8_f32(p[2], p[3], word, true));
            }
#pragma unroll
            for (int ds = 0; ds < 4; ++ds) {
                const uint8_t* src = V + ds * 2048 + rowoff;
                const uint4 v0 = *reinterpret_cast<const uint4*>(src + vq0), v1 = *reinterpret_cast<const uint4*>(src + vq1);
                const i32x8 vf = {int(v0.x), int(v0.y), int(v0.z), int(v0.w), int(v1.x), int(v1.y), int(v1.z), int(v1.w)};
                o[ds] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(vf, pf, o[ds], 0, 0, 0, 0, 0, 0);
            }
            const i32x8 ones = {ONES_E4M3, ONES_E4M3, ONES_E4M3, ONES_E4M3, ONES_E4M3, ONES_E4M3, ONES_E4M3, ONES_E4M3};
            lv = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(ones, pf, lv, 0, 0, 0, 0, 0, 0);
        };

#pragma unroll
        for (int k = 0; k < STAGES - 1; ++k) issue(k, k);
        float qs;
        if (a.qb) {
            // Sage's per-thread int8 Q from bf16, the rule of quant_q_kernel: the wave's 32 queries are one 32-token
            // block, and the group of query q is the 4 tokens with its q % 8 (lanes l, l ^ 8, l ^ 16, l ^ 24 of a
            // half, both halves): scale = max|x| / 127 + 1e-7, q = trunc(x / scale +- 0.5)
            float x[4][16];
            float amax = 0.0f;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                uint4 r0 = make_uint4(0, 0, 0, 0), r1 = r0;
                if (qlive) {
                    const uint16_t* src = a.qb + q * a.ldq + h * D + 32 * c + 16 * half;
                    r0 = *reinterpret_cast<const uint4*>(src);
                    r1 = *reinterpret_cast<const uint4*>(src + 8);
                }
                const uint32_t w[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    x[c][2 * e] = __uint_as_float(w[e] << 16);
                    x[c][2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
                    amax = fmaxf(amax, fmaxf(fabsf(x[c][2 * e]), fabsf(x[c][2 * e + 1])));
                }
            }
            amax = xor_max<32>(xor_max<16>(xor_max<8>(amax)));
            const float scale = amax / 127.0f + 1e-7f;
            // x / scale through the reciprocal (div_rn: the IEEE quotient wherever |x / scale| >= 2^-126, and below
            // that both round to a zero code)
            const float rscale = 1.0f / scale;
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                int wv[4];
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    uint32_t word = 0;
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        const float y = div_rn(x[c][4 * b + e], scale, rscale);
                        const float r = __builtin_truncf(y + (y >= 0.0f ? 0.5f : -0.5f));
                        word |= (uint32_t(int32_t(r)) & 0xffu) << (8 * e);
                    }
                    wv[b] = int(word);
                }
                qf[c] = i32x4{wv[0], wv[1], wv[2], wv[3]};
            }
            qs = qlive ? scale : 0.0f;
        } else {
#pragma unroll
            for (int c = 0; c < 4; ++c) {
                if (qlive) {
                    const uint4 r = *reinterpret_cast<const uint4*>(a.q + q * a.ldq + h * D + 32 * c + 16 * half);
                    qf[c] = i32x4{int(r.x), int(r.y), int(r.z), int(r.w)};
                } else {
                    qf[c] = i32x4{0, 0, 0, 0};
                }
            }
            qs = qlive ? a.q_scale[h * qblocks8 + (q / 32) * 8 + q % 8] : 0.0f;
        }
        cq = qs * a.sm_scale_log2;
        if (new_head) {  // read only after the first ring step's barrier
#pragma unroll
            for (int i = 0; i < KS_MAX / 256; ++i)
                if (tg + 256 * i < nks) sKs[tg + 256 * i] = ksr[i];
            if (tg < D) sVs[tg] = vsr;
            head_loaded = h;
        }
        // ring step i: wait for block i, refill the stage block i - 1 used, compute block i (the group's blocks
        // before fet unmasked, the rest masked: two loops, so each holds only its own variant's registers)
        auto step = [&](int i, auto mask_tag) {
            wait_vmcnt<(STAGES - 2) * LPB>();
            __syncthreads();
            const int st = i % STAGES;
            issue((st + STAGES - 1) % STAGES, i + STAGES - 1);
            if (i < count) compute(st, first + i, mask_tag);
        };
        const int split = fet - first < 0 ? 0 : (fet - first < iters ? fet - first : iters);
        for (int i = 0; i < split; ++i) step(i, std::false_type{});
        for (int i = split; i < iters; ++i) step(i, std::true_type{});
        wait_vmcnt<0>();
        __syncthreads();  // all loads landed, every wave is done with the ring, sKs written

        // group 1 hands (O, m, l) to group 0, which merges: O = O0 2^(m0 - m) + O1 2^(m1 - m), l likewise
        if (grp == 1 && !dualwg) {
#pragma unroll
            for (int ds = 0; ds < 4; ++ds)
#pragma unroll
                for (int e = 0; e < 16; ++e) xo[(ds * 16 + e) * 64 + lane] = o[ds][e];
            xo[64 * 64 + lane] = m;
            xo[64 * 64 + 64 + lane] = lv[0];
        }
        __syncthreads();
        float lt = 0.0f;
        if (dualwg) {
            lt = lv[0];
        } else if (grp == 0) {
            const float m1 = xo[64 * 64 + lane], l1 = xo[64 * 64 + 64 + lane];
            const float mt = fmaxf(m, m1);
            const float a0 = __builtin_amdgcn_exp2f(m - mt), a1 = __builtin_amdgcn_exp2f(m1 - mt);
            lt = lv[0] * a0 + l1 * a1;
#pragma unroll
            for (int ds = 0; ds < 4; ++ds)
#pragma unroll
                for (int e = 0; e < 16; ++e) o[ds][e] = o[ds][e] * a0 + xo[(ds * 16 + e) * 64 + lane] * a1;
            m = mt;
        }

        // out = O / l * v_scale, bf16; lane half h holds channels 32 ds + 8 g + 4 h + e
        // The wave's 32 x 128 bf16 outputs go through its own LDS area (the hand-over slot it has just read, or for a
        // dual workgroup a slot per wave of the ring, which every wave is done with), rows of 272 bytes, and leave as
        // whole 256-byte query rows: 16 bytes per lane, four rows per store instead of 32 rows in 8-byte pieces.
        auto write_out = [&](const f32x16 (&ov)[4], float lsum) {
            const float inv = 1.0f / lsum;
            constexpr int SROW = 136;  // staged row, in bf16 elements (128 + 8 pad)
            static_assert(32 * SROW * 2 <= (64 * 64 + 128) * 4 && 8 * 32 * SROW * 2 <= STAGES * STAGE, "staging");
            uint16_t* stg = dualwg ? reinterpret_cast<uint16_t*>(smem) + (grp * 4 + sub) * 32 * SROW
                                   : reinterpret_cast<uint16_t*>(xo);
#pragma unroll
            for (int ds = 0; ds < 4; ++ds) {
#pragma unroll
                for (int g = 0; g < 4; ++g) {
                    const int d = 32 * ds + 8 * g + 4 * half;
                    uint16_t r[4];
#pragma unroll
                    for (int e = 0; e < 4; ++e) r[e] = f32_to_bf16(ov[ds][4 * g + e] * inv * sVs[d + e]);
                    *reinterpret_cast<uint2*>(stg + (lane % 32) * SROW + d) =
                        make_uint2(r[0] | (uint32_t(r[1]) << 16), r[2] | (uint32_t(r[3]) << 16));
                }
            }
            const int64_t q0 = qt * 128 + sub * 32;  // the wave's first query
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = 4 * i + lane / 16, c = lane % 16;
                const uint4 v = *reinterpret_cast<const uint4*>(stg + row * SROW + 8 * c);
                if (q0 + row < a.n) *reinterpret_cast<uint4*>(a.out + (q0 + row) * a.ldo + h * D + 8 * c) = v;
            }
        };

        if (slot < 0) {
            if (grp == 0 || dualwg) write_out(o, lt);
        } else if (grp == 0) {
            float* ps = a.part + slot * SLOT_FLOATS + sub * (64 * 64 + 128);
#pragma unroll
            for (int ds = 0; ds < 4; ++ds)
#pragma unroll
                for (int e = 0; e < 16; ++e) ps[(ds * 16 + e) * 64 + lane] = o[ds][e];
            ps[64 * 64 + lane] = m;
            ps[64 * 64 + 64 + lane] = lt;
        }
        __syncthreads();  // the segment is done with the ring, the hand-over area, sKs and sVs
    }
}

// The split tiles: tile D + r gathers the partial states of the workgroups whose key-block share meets it, in
// workgroup order: m = max_c m_c, O = sum_c O_c 2^(m_c - m), l = sum_c l_c 2^(m_c - m), out = O / l * v_scale.
// Grid (R, 4 query waves, 4 channel subtiles) x 256 threads: lane = query (and channel half), thread / 64 = one
// group of 4 channels, in the partial layout of the main kernel.
__global__ __launch_bounds__(256) void attn_merge_kernel(AttnArgs a) {
    const int lane = threadIdx.x % 64, half = lane / 32, g = __builtin_amdgcn_readfirstlane(threadIdx.x / 64);
    const int64_t r = blockIdx.x, sub = blockIdx.y, ds = blockIdx.z;
    const int64_t nblk = a.Lpad / 64, T = a.qtiles * a.H, Usk = (T - a.D) * nblk;
    const int64_t tile = a.D + r, h = tile / a.qtiles, qt = tile % a.qtiles;
    const int64_t q = qt * 128 + sub * 32 + lane % 32;
    const int64_t cf = wg_of(r * nblk, Usk, a.Wt), cl = wg_of((r + 1) * nblk - 1, Usk, a.Wt);
    // the contributors' slots, once per workgroup (one thread each): slot 2c if the tile is c's first piece, 2c + 1
    // if its second, -1 if c's share is empty (fewer split key blocks than workgroups). Share starts in 32-bit
    // arithmetic (the host keeps W * Usk below 2^31).
    __shared__ int cslot[MAX_WG];
    const uint32_t Uu = uint32_t(Usk), Wu = uint32_t(a.Wt), tile0 = uint32_t(r * nblk);
    const int nc = int(cl - cf + 1);
    for (int i = threadIdx.x; i < nc; i += 256) {
        const uint32_t c = uint32_t(cf) + i, s0 = c * Uu / Wu, s1 = (c + 1) * Uu / Wu;
        cslot[i] = s0 == s1 ? -1 : int(s0 >= tile0 ? 2 * c : 2 * c + 1);
    }
    __syncthreads();
    auto part = [&](int slot) { return a.part + int64_t(slot) * SLOT_FLOATS + sub * (64 * 64 + 128); };
    // contributors in batches with all their loads issued together (one memory round trip per batch)
    constexpr int BATCH = 16, MBATCH = 32;
    float mt = -INFINITY;
    for (int i0 = 0; i0 < nc; i0 += MBATCH) {
        float mv[MBATCH];
#pragma unroll
        for (int k = 0; k < MBATCH; ++k) {
            const int sl = i0 + k < nc ? cslot[i0 + k] : -1;
            mv[k] = sl >= 0 ? part(sl)[64 * 64 + lane] : -INFINITY;
        }
#pragma unroll
        for (int k = 0; k < MBATCH; ++k) mt = fmaxf(mt, mv[k]);
    }
    float ov[4] = {}, ls = 0.0f;
    for (int i0 = 0; i0 < nc; i0 += BATCH) {
        float mv[BATCH], lv[BATCH], pv[BATCH][4];
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
            const int sl = i0 + k < nc ? cslot[i0 + k] : -1;
            const float* ps = part(sl >= 0 ? sl : cslot[0]);  // contributor cf always has a piece of the tile
            mv[k] = sl >= 0 ? ps[64 * 64 + lane] : -INFINITY;
            lv[k] = ps[64 * 64 + 64 + lane];
#pragma unroll
            for (int e = 0; e < 4; ++e) pv[k][e] = ps[(ds * 16 + 4 * g + e) * 64 + lane];
        }
#pragma unroll
        for (int k = 0; k < BATCH; ++k) {
            const float f = __builtin_amdgcn_exp2f(mv[k] - mt);  // 0 for an absent contributor
            ls = ls + lv[k] * f;
#pragma unroll
            for (int e = 0; e < 4; ++e) ov[e] = ov[e] + pv[k][e] * f;
        }
    }
    if (q >= a.n) return;
    const float inv = 1.0f / ls;
    const int d = 32 * int(ds) + 8 * g + 4 * half;
    uint16_t rr[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) rr[e] = f32_to_bf16(ov[e] * inv * a.v_scale[h * D + d + e]);
    *reinterpret_cast<uint2*>(a.out + q * a.ldo + h * D + d) =
        make_uint2(rr[0] | (uint32_t(rr[1]) << 16), rr[2] | (uint32_t(rr[3]) << 16));
}

}  // namespace


// workspace: [2 W][SLOT_FLOATS] fp32 partial states, W <= T (query tiles x heads)
extern "C" int64_t wdl_sage_attn_workspace_bytes(int64_t n, int64_t L, int64_t heads) {
    if (n <= 0 || L < 1 || heads <= 0) return 0;
    const int64_t T = (n + 127) / 128 * heads;
    return 2 * T * SLOT_FLOATS * 4;
}

static int attn_launch(const void* q_i8, const float* q_scale, const void* q_bf16, int64_t ldq, const void* k_i8,
                       const float* k_scale, const void* v_fp8, const float* v_scale, int64_t n, int64_t L,
                       int64_t heads, float sm_scale, void* out, int64_t ldo, void* workspace, hipStream_t stream,
                       int64_t frame = 0) {
    const void* q = q_bf16 ? q_bf16 : q_i8;
    const int64_t qbytes = q_bf16 ? 2 : 1;
    if (n < 0 || L < 1 || heads <= 0 || ldq < heads * D || ldo < heads * D)
        return fail(WDL_EINVAL, "sage_attn: bad shape n=%lld L=%lld", (long long)n, (long long)L);
    if (!q || (!q_bf16 && !q_scale) || !k_i8 || !k_scale || !v_fp8 || !v_scale || !out)
        return fail(WDL_EINVAL, "sage_attn: null pointer");
    if ((reinterpret_cast<uintptr_t>(q) | reinterpret_cast<uintptr_t>(out) | (ldq * qbytes) | (ldo * 2)) % 16)
        return fail(WDL_EINVAL, "sage_attn: unaligned rows");
    if (frame < 0 || (frame > 0 && n > L))
        return fail(WDL_EINVAL, "sage_attn: frame=%lld needs the n=%lld queries' own keys among the L=%lld",
                    (long long)frame, (long long)n, (long long)L);
    if (n == 0) return WDL_OK;
    const int64_t Lpad = (L + 63) / 64 * 64;
    if (Lpad / 16 > KS_MAX) return fail(WDL_EINVAL, "sage_attn: L=%lld above %d keys", (long long)L, KS_MAX * 16);
    if ((reinterpret_cast<uintptr_t>(k_i8) | reinterpret_cast<uintptr_t>(v_fp8)) % 16)
        return fail(WDL_EINVAL, "sage_attn: K / V must be 16-byte aligned");
    const int64_t qtiles = (n + 127) / 128, T = qtiles * heads, nblk = Lpad / 64;
    // One workgroup per tile, unless that leaves a large share of the last round of CUs idle (tiles just above a
    // multiple of the CU count): then one workgroup per CU runs floor(T / CUs) whole tiles each and the key blocks
    // of the T mod CUs remaining tiles are split evenly over all of them, merged by a second launch. Short key
    // ranges keep one workgroup per tile.
    // Short key ranges (no split) with CUs < T <= 2 CUs: one workgroup per CU, and the first T - CUs of them run
    // two whole tiles, one per group of 4 waves over all the key blocks (the other workgroups split their tile's
    // blocks between the groups), so the tiles take one round instead of two.
    int64_t W = T, Dw = T, dual = 0;
    const int64_t cus = cu_count();
    // (under the per-frame mask tiles differ in key count: none is split)
    if (frame == 0 && cus > 0 && cus <= MAX_WG && T > cus && nblk >= 32) {
        const int64_t rounds = (T + cus - 1) / cus;
        const int64_t usk = (T % cus) * nblk;  // key blocks of the split tiles
        if (T * 100 < 85 * rounds * cus && (cus + 1) * usk < (int64_t(1) << 31)) W = cus, Dw = cus * (T / cus);
    } else if (cus > 0 && T > cus && T <= 2 * cus && (nblk < 32 || cus > MAX_WG)) {
        W = cus, dual = T - cus;
    }
    if (Dw < T && (!workspace || reinterpret_cast<uintptr_t>(workspace) % 16))
        return fail(WDL_EINVAL, "sage_attn: a 16-byte aligned workspace of wdl_sage_attn_workspace_bytes is needed");
    float* part = Dw < T ? static_cast<float*>(workspace) : nullptr;
    AttnArgs a{static_cast<const int8_t*>(q_i8), ldq, q_scale, static_cast<const int8_t*>(k_i8), k_scale,
               static_cast<const uint8_t*>(v_fp8), v_scale, static_cast<uint16_t*>(out), ldo, n, L, Lpad, heads,
               sm_scale * 1.4426950408889634f, part, W, qtiles, Dw, static_cast<const uint16_t*>(q_bf16), dual,
               W / TAIL_DIV > 0 ? W / TAIL_DIV : 1, frame};
    sage_attn_kernel<<<unsigned(W), 512, 0, stream>>>(a);
    int rc = check_launch("sage_attn");
    if (rc || Dw == T) return rc;
    attn_merge_kernel<<<dim3(unsigned(T - Dw), 4, 4), 256, 0, stream>>>(a);
    return check_launch("sage_attn merge");
}

extern "C" int wdl_sage_attn(const void* q_i8, int64_t ldq, const float* q_scale, const void* k_i8,
                             const float* k_scale, const void* v_fp8, const float* v_scale, int64_t n, int64_t L,
                             int64_t heads, float sm_scale, void* out, int64_t ldo, void* workspace,
                             hipStream_t stream) {
    if (!q_i8) return fail(WDL_EINVAL, "sage_attn: null pointer");
    return attn_launch(q_i8, q_scale, nullptr, ldq, k_i8, k_scale, v_fp8, v_scale, n, L, heads, sm_scale, out, ldo,
                       workspace, stream);
}

extern "C" int wdl_sage_attn_q16(const void* q_bf16, int64_t ldq, const void* k_i8, const float* k_scale,
                                 const void* v_fp8, const float* v_scale, int64_t n, int64_t L, int64_t heads,
                                 float sm_scale, void* out, int64_t ldo, void* workspace, hipStream_t stream) {
    if (!q_bf16) return fail(WDL_EINVAL, "sage_attn_q16: null pointer");
    return attn_launch(nullptr, nullptr, q_bf16, ldq, k_i8, k_scale, v_fp8, v_scale, n, L, heads, sm_scale, out, ldo,
                       workspace, stream);
}

extern "C" int wdl_sage_attn_q16_framed(const void* q_bf16, int64_t ldq, const void* k_i8, const float* k_scale,
                                        const void* v_fp8, const float* v_scale, int64_t n, int64_t L, int64_t heads,
                                        float sm_scale, int64_t frame_tokens, void* out, int64_t ldo,
                                        void* workspace, hipStream_t stream) {
    if (!q_bf16) return fail(WDL_EINVAL, "sage_attn_q16_framed: null pointer");
    if (frame_tokens <= 0) return fail(WDL_EINVAL, "sage_attn_q16_framed: frame_tokens must be positive");
    return attn_launch(nullptr, nullptr, q_bf16, ldq, k_i8, k_scale, v_fp8, v_scale, n, L, heads, sm_scale, out, ldo,
                       workspace, stream, frame_tokens);
}
