// Per-token, per-64-channel activation quantizer of the W4A4 linears, optionally fused with the LayerNorm and the
// adaLN modulation that precede it, and with the down projection of the low-rank branch.
//
// For rows m < M of x (bf16 [M, K], row stride ldx):
//   v     = x                                                       (plain), or
//   v     = bf16( LN(x)[*w + b] * (1 + mod_scale) + mod_shift )    (fused; fp32 math, one rounding)
//   u     = (v + qshift) / smooth                                   (IEEE fp32 quotient)
//   scale = bf16( max_{64 group} |u| / qmax )                       (qmax 7 signed, 15 unsigned)
//   q     = clamp(rint(u / scale))                                  (0 where scale is 0)
//   lora  = v . proj_down                                           (bf16 MFMA, fp32 sums)
// Outputs: q as fp6 codes (e2m3 of q / 2, exact) [Mp, K] (rows >= M zero) in the W4A4 GEMM's tile-blocked layout
// ([Mp / 128][K / 64][128][48 bytes], Mp a multiple of 128; see blocked6_offset); ascales bf16 [K/64, Mp]; lora
// fp32 [Mp, 32].
//
// LayerNorm statistics come from per-chunk partials of x: for each row and 32-value chunk c, (S_c, M2_c) = the
// chunk's sum and its sum of squared deviations from its own mean, each as 8 quads summed sequentially and the
// quads combined as ((t0 + t1) + (t2 + t3)) + ((t4 + t5) + (t6 + t7)). The W4A4 GEMM's gated-residual epilogue
// writes them for the rows it produces (wdl_w4a4_gemm's ln_partials), in the same order; otherwise ln_partials
// runs here. The quant launch merges a row's C = K / 32 chunks over 8 lanes (lane j: the chunk pairs j, j + 8, ...
// — chunks 2p, 2p + 1, one 16-byte load each — in chunk order from +0, the lanes combined by an xor butterfly 1, 2,
// 4): mean = sum S_c / K, M2 = sum of
// M2_c + 32 (S_c / 32 - mean)^2, var = M2 / K, rstd = 1 / sqrt(var + eps).
//
// Launches (all parallel over rows and column blocks, nothing serial over K):
//   ln_partials (LN only, when the caller passes no partials): one thread per (row, chunk).
//   quant      grid (Mp / 32, ceil(K / 64 / S)): 32 rows x S 64-groups per workgroup of S waves (S = 4 up to
//              K = 4096, 8 above), each wave one group of the 32 rows; lane l owns row l % 32 and half
//              l / 32 of a group (64 bytes of x, loaded up front with the matching 64 bytes of proj_down^T); the
//              group maximum is one exchange between lanes l and l ^ 32, the codes of a half are packed by one
//              hardware fp6 conversion and written with two aligned stores, and the low-rank product runs on the
//              values in registers (bf16 MFMA), the waves' 32 x 32 partials summed in wave order.
//   lora_sum   lora = sum of the column-block partials in increasing order (only when K / 64 > S).
#include <mutex>

#include "wdl_common.h"

namespace {

using namespace wdl;

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef unsigned u32x6 __attribute__((ext_vector_type(6)));

constexpr int ROWS = 32;
constexpr int RANK = 32;
// Shape of the quant launch's workgroups: WAVES waves on 32 rows, G 64-groups per wave (S = WAVES * G groups per
// workgroup), one shape up to K = 4096 and one above. Measured at 1392 rows: 4 x 1 at K = 3072 (10.0 us; 8 x 1,
// 4 x 2 and 16 x 1 take 10.8 - 12.6 us), 8 x 1 at K = 14336 (22.1 us; 8 x 2, 4 x 2 and 16 x 1 take 25 - 33 us).
constexpr int SMALL_WAVES = 4, SMALL_G = 1, BIG_WAVES = 8, BIG_G = 1;
constexpr int groups_per_block(int64_t K) { return K <= 4096 ? SMALL_WAVES * SMALL_G : BIG_WAVES * BIG_G; }
constexpr int MAXCH = 8; // LN rows: K <= 64 * 8 * MAXCH = 4096 (the merge holds up to 16 chunks per lane)
constexpr int LN_CHUNK = 32;

__device__ __forceinline__ void load8(const uint16_t* p, float* f) {
    uint4 raw = *reinterpret_cast<const uint4*>(p);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        f[2 * j] = __uint_as_float(w[j] << 16);
        f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
    }
}

// ((t0 + t1) + (t2 + t3)) + ((t4 + t5) + (t6 + t7)) of the 8 quad sums of a chunk
__device__ __forceinline__ float tree8(const float* t) {
    return ((t[0] + t[1]) + (t[2] + t[3])) + ((t[4] + t[5]) + (t[6] + t[7]));
}

// (S_c, M2_c) of one 32-value chunk held in registers
__device__ __forceinline__ float2 chunk_partial(const float* v) {
    float t[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) t[k] = ((v[4 * k] + v[4 * k + 1]) + v[4 * k + 2]) + v[4 * k + 3];
    const float S = tree8(t), mc = S * (1.0f / LN_CHUNK);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const float d0 = v[4 * k] - mc, d1 = v[4 * k + 1] - mc, d2 = v[4 * k + 2] - mc, d3 = v[4 * k + 3] - mc;
        t[k] = ((d0 * d0 + d1 * d1) + d2 * d2) + d3 * d3;
    }
    return make_float2(S, tree8(t));
}

// LayerNorm chunk partials of x [M, K]: thread = (row, chunk), part [M][K / 32]
__global__ __launch_bounds__(256) void ln_partials_kernel(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                                                          float2* part) {
    const int64_t C = K / LN_CHUNK, i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= M * C) return;
    const int64_t row = i / C, c = i % C;
    float v[LN_CHUNK];
#pragma unroll
    for (int j = 0; j < 4; ++j) load8(x + row * ldx + c * LN_CHUNK + 8 * j, v + 8 * j);
    part[i] = chunk_partial(v);
}

struct QuantArgs {
    const uint16_t* x;
    int64_t ldx;
    int64_t M, Mp, K;
    const uint16_t* smooth;    // bf16 [K]
    float qshift;
    int unsigned_q;
    const uint16_t* pdt;       // bf16 [RANK, K] (proj_down transposed), or null (no low-rank branch)
    uint8_t* q;                // [Mp, K], tile-blocked
    uint16_t* ascales;         // [K/64, Mp]
    float* lora;               // [nblocks, Mp, RANK] partials (or [Mp, RANK] when nblocks == 1)
    const float2* lnp;         // LN chunk partials [M][K / 32] (LN rows), or null (no LN)
    const float* mod_shift;    // fp32 [K] or null
    const float* mod_scale;    // fp32 [K] or null (used as 1 + scale)
    const float* ln_w;         // fp32 [K] or null
    const float* ln_b;         // fp32 [K] or null
    uint16_t* v_out;           // bf16 [M, K] copy of v, or null
    float eps;                 // LN
};

// Workgroups of WAVES waves on the same 32 rows; wave w takes the 64-groups w, w + WAVES, ... (G of them) of the
// workgroup's S = WAVES * G groups. Lane l of a wave owns row l % 32 and half h = l / 32 of each of its groups (32
// columns, 64 bytes of x): the group maximum is one exchange with lane l ^ 32, the 32 codes of the half are one
// hardware fp6 conversion, and the 32 lanes of a half write the 48-byte group rows of 32 consecutive tokens (1.5 KB
// contiguous in the tile-blocked layout). The lane's bf16 values are also the A operand of the low-rank MFMA
// (32 x 32 x 16: lane l supplies row l % 32 and k-slots 8h..8h+7, here columns 32h + 8s .. 32h + 8s + 7 of the
// group for the s-th of its 4 MFMAs) and the B operand comes from proj_down^T with the same column map, so the
// product needs no LDS tile; the waves' 32 x 32 partials are summed in wave order through LDS at the end.
template <int WAVES, int G, bool LN>
__global__ __launch_bounds__(64 * WAVES) void quant_kernel(QuantArgs a) {
    constexpr int S = WAVES * G, NT = 64 * WAVES, SC = 64 * S;  // groups, threads and columns of the workgroup
    // per-column vectors of the workgroup's columns: smooth, LN weight, LN bias, 1 + mod_scale, mod_shift,
    // 1 / smooth
    __shared__ __attribute__((aligned(16))) float sp[6][SC];
    __shared__ float part[WAVES][ROWS * RANK];
    __shared__ float2 sst[LN ? ROWS : 1];  // LN (mean, rstd) of the workgroup's rows

    const int t = threadIdx.x, lane = t % 64, wave = __builtin_amdgcn_readfirstlane(t / 64);  // uniform: scalar
    const int r = lane % 32, h = lane / 32;
    const int64_t row = int64_t(blockIdx.x) * ROWS + r;
    const bool live = row < a.M;
    const int64_t K = a.K;
    const int64_t gb = int64_t(blockIdx.y) * S;             // first group of the workgroup
    const int nsg = int(min(int64_t(S), K / 64 - gb));     // its groups present in the matrix

    // loads first: each present group's 64 bytes of the row (absent rows read row 0: every output of theirs is
    // masked below, the codes and scales by their store, the low-rank sums by the partial store) and of
    // proj_down^T row r, the row's LN statistics, the workgroup's per-column vectors (thread t: columns t + NT i)
    uint4 raw[G][4], pd[G][4];
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const int gl = wave + WAVES * j;
        if (gl >= nsg) continue;  // uniform over the wave
        const int64_t col = (gb + gl) * 64 + 32 * h;
        if (a.M > 0) {
            const uint16_t* xr = a.x + (live ? row : 0) * a.ldx + col;
#pragma unroll
            for (int i = 0; i < 4; ++i) raw[j][i] = *reinterpret_cast<const uint4*>(xr + 8 * i);
        } else {
#pragma unroll
            for (int i = 0; i < 4; ++i) raw[j][i] = make_uint4(0u, 0u, 0u, 0u);
        }
        if (a.pdt) {
            const uint16_t* pr = a.pdt + int64_t(r) * K + col;
#pragma unroll
            for (int i = 0; i < 4; ++i) pd[j][i] = *reinterpret_cast<const uint4*>(pr + 8 * i);
        }
    }
    // LN: this lane's merge slot — row 8 wave + lane / 8 of the workgroup, the chunk pairs j, j + 8, ... of it
    // (j = lane % 8; C is even since K % 64 == 0), loaded with the row data
    constexpr int MAXCP = 64 * 8 * MAXCH / LN_CHUNK / 8;  // chunks per slot at K = 4096
    float2 cp[LN ? MAXCP : 1];
    int ncp = 0;
    if constexpr (LN) {
        static_assert(WAVES * 8 == ROWS, "the merge maps the workgroup's rows to its waves, 8 rows x 8 slots each");
        const int64_t C = K / LN_CHUNK, mrow = int64_t(blockIdx.x) * ROWS + 8 * wave + lane / 8;
        const int j = lane % 8;
        ncp = 2 * int((C / 2 - j + 7) / 8);
#pragma unroll
        for (int i = 0; i < MAXCP / 2; ++i) {
            float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            if (2 * i < ncp && mrow < a.M)
                v = *reinterpret_cast<const float4*>(a.lnp + mrow * C + 2 * (j + 8 * i));
            cp[2 * i] = make_float2(v.x, v.y);
            cp[2 * i + 1] = make_float2(v.z, v.w);
        }
    }
#pragma unroll
    for (int i = 0; i < G; ++i) {
        const int c = t + NT * i;
        if (c >= nsg * 64) continue;
        const int64_t cg = gb * 64 + c;
        const float sm = bf16_to_f32(a.smooth[cg]);
        // an absent LN weight / modulation scale is x 1 and an absent bias / shift is + (-0): exact identities
        // (x + -0 = x for every x, signed zeros included), so the LayerNorm below needs no per-value branches
        float p1 = 1.0f, p2 = -0.0f, p3 = 1.0f, p4 = -0.0f;
        if (LN) {
            if (a.ln_w) p1 = a.ln_w[cg];
            if (a.ln_b) p2 = a.ln_b[cg];
            if (a.mod_scale) p3 = 1.0f + a.mod_scale[cg];
            if (a.mod_shift) p4 = a.mod_shift[cg];
        }
        sp[0][c] = sm;
        sp[1][c] = p1;
        sp[2][c] = p2;
        sp[3][c] = p3;
        sp[4][c] = p4;
        sp[5][c] = 1.0f / sm;
    }
    if constexpr (LN) {  // the row's (mean, rstd) from its chunk partials, into sst
        float sum = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXCP; ++i)
            if (i < ncp) sum = sum + cp[i].x;
        sum = xor_sum<4>(xor_sum<2>(xor_sum<1>(sum)));
        const float mean = sum / float(K);
        float m2 = 0.0f;
#pragma unroll
        for (int i = 0; i < MAXCP; ++i)
            if (i < ncp) {
                const float d = cp[i].x * (1.0f / LN_CHUNK) - mean;
                m2 = m2 + (cp[i].y + float(LN_CHUNK) * (d * d));
            }
        m2 = xor_sum<4>(xor_sum<2>(xor_sum<1>(m2)));
        if (lane % 8 == 0) sst[8 * wave + lane / 8] = make_float2(mean, 1.0f / sqrtf(m2 / float(K) + a.eps));
    }
    __syncthreads();
    const float2 st = (LN && live) ? sst[r] : make_float2(0.0f, 0.0f);

    const float qmax = a.unsigned_q ? 15.0f : 7.0f;
    const float qlo = a.unsigned_q ? 0.0f : -8.0f;
    f32x16 acc = {};
#pragma unroll
    for (int j = 0; j < G; ++j) {
        const int gl = wave + WAVES * j;
        if (gl >= nsg) continue;
        const int cl = 64 * gl + 32 * h;  // the lane's first column in the workgroup
        float v[32];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w[4] = {raw[j][i].x, raw[j][i].y, raw[j][i].z, raw[j][i].w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                v[8 * i + 2 * e] = __uint_as_float(w[e] << 16);
                v[8 * i + 2 * e + 1] = __uint_as_float(w[e] & 0xffff0000u);
            }
        }
        if (LN) {  // rows past M compute with (0, 0) statistics; their outputs are masked
#pragma unroll
            for (int j4 = 0; j4 < 8; ++j4) {
                const float4 w4 = *reinterpret_cast<const float4*>(&sp[1][cl + 4 * j4]);
                const float4 b4 = *reinterpret_cast<const float4*>(&sp[2][cl + 4 * j4]);
                const float4 s4 = *reinterpret_cast<const float4*>(&sp[3][cl + 4 * j4]);
                const float4 h4 = *reinterpret_cast<const float4*>(&sp[4][cl + 4 * j4]);
                const float wv[4] = {w4.x, w4.y, w4.z, w4.w}, bv4[4] = {b4.x, b4.y, b4.z, b4.w};
                const float sv[4] = {s4.x, s4.y, s4.z, s4.w}, hv[4] = {h4.x, h4.y, h4.z, h4.w};
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int k = 4 * j4 + e;
                    float n = (v[k] - st.x) * st.y;
                    n = n * wv[e];
                    n = n + bv4[e];
                    n = n * sv[e];
                    n = n + hv[e];
                    v[k] = bf16_to_f32(f32_to_bf16(n));
                }
            }
        }
        // v is bf16-valued here: its top 16 bits, packed in pairs, are the MFMA operand and the v_out row
        const int64_t g = gb + gl;
        uint32_t pw[16];
#pragma unroll
        for (int k = 0; k < 16; ++k)
            pw[k] = (__float_as_uint(v[2 * k]) >> 16) | (__float_as_uint(v[2 * k + 1]) & 0xffff0000u);
        if (a.v_out && live) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<uint4*>(a.v_out + row * K + g * 64 + 32 * h + 8 * i) =
                    make_uint4(pw[4 * i], pw[4 * i + 1], pw[4 * i + 2], pw[4 * i + 3]);
        }
        if (a.pdt) {
#pragma unroll
            for (int s8 = 0; s8 < 4; ++s8) {
                const uint4 av = make_uint4(pw[4 * s8], pw[4 * s8 + 1], pw[4 * s8 + 2], pw[4 * s8 + 3]);
                acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, av),
                                                              __builtin_bit_cast(bf16x8, pd[j][s8]), acc, 0, 0, 0);
            }
        }
        float u[32];
        float amax = 0.0f;
#pragma unroll
        for (int j4 = 0; j4 < 8; ++j4) {
            const float4 d4 = *reinterpret_cast<const float4*>(&sp[0][cl + 4 * j4]);
            const float4 r4 = *reinterpret_cast<const float4*>(&sp[5][cl + 4 * j4]);
            const float dv[4] = {d4.x, d4.y, d4.z, d4.w}, rv[4] = {r4.x, r4.y, r4.z, r4.w};
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const int k = 4 * j4 + e;
                u[k] = div_rn(v[k] + a.qshift, dv[e], rv[e]);
                amax = fmaxf(amax, fabsf(u[k]));
            }
        }
        amax = xor_max<32>(amax);  // the group's other half
        const uint16_t sb = f32_to_bf16(amax / qmax);
        const float sc = bf16_to_f32(sb);
        const float rsc = sc > 0.0f ? 1.0f / sc : 0.0f;
        // fp6 codes of q / 2 (e2m3, exact): even positions go in the first operand, odd in the second, because
        // the conversion places element i of its first operand in field 2i and of its second in field 2i + 1
        f32x16 ea, eb;
#pragma unroll
        for (int k = 0; k < 32; ++k) {
            const float rq = sc > 0.0f ? __builtin_rintf(div_rn(u[k], sc, rsc)) : 0.0f;
            const float qv = fminf(fmaxf(rq, qlo), qmax) + 0.0f;  // + 0 turns -0 into +0
            if (k % 2 == 0) ea[k / 2] = qv * 0.5f;
            else eb[k / 2] = qv * 0.5f;
        }
        // early-clobber output: the instruction writes its first result dwords before it has read all of its
        // sources, and the builtin lets the compiler place the result over the first operand (which corrupted
        // field 4, measured); scale 1.0 (the values are exact fp6 values)
        u32x6 w;
        asm volatile("v_cvt_scalef32_2xpk16_fp6_f32 %0, %1, %2, 1.0" : "=&v"(w) : "v"(ea), "v"(eb));
#pragma unroll
        for (int d = 0; d < 6; ++d) w[d] = live ? w[d] : 0u;  // rows past M: code 0 (+0) everywhere
        uint8_t* dst = a.q + blocked6_offset(row, g, K);
        *reinterpret_cast<uint4*>(dst + 16 * h) = make_uint4(w[0], w[1], w[2], w[3]);
        *reinterpret_cast<uint2*>(dst + 32 + 8 * h) = make_uint2(w[4], w[5]);
        if (h == 0) a.ascales[g * a.Mp + row] = live ? sb : uint16_t(0);
    }
    if (!a.pdt) return;
    // lane l holds the partial of token 8 (i / 4) + 4 h + i % 4 and rank r in acc[i]
#pragma unroll
    for (int i = 0; i < 16; ++i) part[wave][(8 * (i / 4) + 4 * h + (i % 4)) * RANK + r] = acc[i];
    __syncthreads();
    float* dst = a.lora + int64_t(blockIdx.y) * a.Mp * RANK;
    for (int e = t; e < ROWS * RANK; e += NT) {
        const int64_t rr = int64_t(blockIdx.x) * ROWS + e / RANK;
        float sum = part[0][e];
#pragma unroll
        for (int w = 1; w < WAVES; ++w) sum = sum + part[w][e];
        dst[rr * RANK + e % RANK] = rr < a.M ? sum : 0.0f;
    }
}

// lora = sum of the nb column-block partials, in increasing block order; the loads of a batch of 16 partials are
// all issued before the first add (one memory round trip per batch, not one per partial)
__global__ void lora_sum_kernel(const float* part, int nb, int64_t n, float* out) {
    const int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x;
    if (i >= n) return;
    constexpr int BATCH = 16;
    float s = 0.0f;
    for (int b0 = 0; b0 < nb; b0 += BATCH) {
        float v[BATCH];
#pragma unroll
        for (int k = 0; k < BATCH; ++k) v[k] = b0 + k < nb ? part[int64_t(b0 + k) * n + i] : 0.0f;
#pragma unroll
        for (int k = 0; k < BATCH; ++k)
            if (b0 + k < nb) s = b0 + k == 0 ? v[k] : s + v[k];
    }
    out[i] = s;
}

// The same sum over many partials (the fused MLP's 112 tile partials): 4 lanes per output, lane j adding the
// partials [j nb / 4, (j + 1) nb / 4) in increasing order, the four sums combined as (s0 + s1) + (s2 + s3) (DPP
// exchanges): a quarter of the dependent load batches per output.
__global__ __launch_bounds__(256) void lora_sum4_kernel(const float* part, int nb, int64_t n, float* out) {
    const int64_t i = int64_t(blockIdx.x) * 64 + threadIdx.x / 4;
    const int j = threadIdx.x % 4;
    const bool live = i < n;  // every lane takes part in the exchanges
    const int b0 = j * nb / 4, b1 = (j + 1) * nb / 4;
    constexpr int BATCH = 16;
    float s = 0.0f;
    for (int c0 = b0; c0 < b1; c0 += BATCH) {
        float v[BATCH];
#pragma unroll
        for (int k = 0; k < BATCH; ++k) v[k] = live && c0 + k < b1 ? part[int64_t(c0 + k) * n + i] : 0.0f;
#pragma unroll
        for (int k = 0; k < BATCH; ++k)
            if (c0 + k < b1) s = c0 + k == b0 ? v[k] : s + v[k];
    }
    s = xor_sum<2>(xor_sum<1>(s));
    if (live && j == 0) out[i] = s;
}

}  // namespace

namespace wdl {

int lora_sum(const float* part, int nb, int64_t n, float* out, hipStream_t stream) {
    if (nb >= 32) {
        lora_sum4_kernel<<<unsigned((n + 63) / 64), 256, 0, stream>>>(part, nb, n, out);
        return check_launch("lora_sum");
    }
    lora_sum_kernel<<<unsigned((n + 255) / 256), 256, 0, stream>>>(part, nb, n, out);
    return check_launch("lora_sum");
}

}  // namespace wdl

extern "C" int64_t wdl_act_quant_workspace_floats(int64_t Mp, int64_t K) {
    const int64_t S = groups_per_block(K), nb = (K / 64 + S - 1) / S;
    // the low-rank column-block partials, then (LN-capable widths) the LayerNorm chunk partials
    return (nb > 1 ? nb * Mp * RANK : 0) + (K <= 64 * 8 * MAXCH ? Mp * (K / LN_CHUNK) * 2 : 0);
}

namespace {

int act_quant_launch(const void* x, int64_t ldx, int64_t M, int64_t K, const void* smooth, float qshift,
                     int unsigned_q, const void* proj_down_t, int64_t rank, void* q, void* ascales, float* lora,
                     int64_t Mp, const float* mod_shift, const float* mod_scale, const float* ln_w, const float* ln_b,
                     int ln, float eps, const float* ln_partials, void* v_out, float* workspace,
                     hipStream_t stream) {
    if (M < 0 || K <= 0 || K % 64 || Mp < M || Mp % BLOCK_ROWS || ldx < K)
        return fail(WDL_EINVAL, "act_quant_w4: bad shape M=%lld K=%lld Mp=%lld ldx=%lld", (long long)M,
                    (long long)K, (long long)Mp, (long long)ldx);
    if (ln && K > 64 * 8 * MAXCH) return fail(WDL_EINVAL, "act_quant_w4: LayerNorm rows above 4096");
    if (proj_down_t && rank != RANK) return fail(WDL_EINVAL, "act_quant_w4: rank %lld != 32", (long long)rank);
    if (!x || !smooth || !q || !ascales || (proj_down_t && !lora) || !workspace)
        return fail(WDL_EINVAL, "act_quant_w4: null pointer");
    if ((reinterpret_cast<uintptr_t>(x) | (ldx * 2)) % 16)
        return fail(WDL_EINVAL, "act_quant_w4: x rows must be 16-byte aligned");
    if (ln_partials && reinterpret_cast<uintptr_t>(ln_partials) % 16)
        return fail(WDL_EINVAL, "act_quant_w4: LayerNorm partials must be 16-byte aligned");
    if (Mp == 0) return WDL_OK;
    const int S = groups_per_block(K), nb = int((K / 64 + S - 1) / S);
    // LayerNorm chunk partials: the caller's (written by the GEMM epilogue that produced x), or made here
    const float2* lnp = reinterpret_cast<const float2*>(ln_partials);
    if (ln && !ln_partials) {
        float2* wp = reinterpret_cast<float2*>(workspace + (nb > 1 ? int64_t(nb) * Mp * RANK : 0));
        if (M > 0) {
            const int64_t n = M * (K / LN_CHUNK);
            ln_partials_kernel<<<unsigned((n + 255) / 256), 256, 0, stream>>>(static_cast<const uint16_t*>(x), ldx,
                                                                               M, K, wp);
            int rc = check_launch("act_quant_w4 ln_partials");
            if (rc) return rc;
        }
        lnp = wp;
    }
    QuantArgs a{static_cast<const uint16_t*>(x), ldx, M, Mp, K, static_cast<const uint16_t*>(smooth), qshift,
                unsigned_q, static_cast<const uint16_t*>(proj_down_t), static_cast<uint8_t*>(q),
                static_cast<uint16_t*>(ascales), nb > 1 ? workspace : lora, ln ? lnp : nullptr, mod_shift,
                mod_scale, ln_w, ln_b, static_cast<uint16_t*>(v_out), eps};
    const dim3 grid(unsigned(Mp / ROWS), unsigned(nb));
    if (K <= 4096) {
        if (ln) quant_kernel<SMALL_WAVES, SMALL_G, true><<<grid, 64 * SMALL_WAVES, 0, stream>>>(a);
        else quant_kernel<SMALL_WAVES, SMALL_G, false><<<grid, 64 * SMALL_WAVES, 0, stream>>>(a);
    } else {  // no LayerNorm at these widths (checked above)
        quant_kernel<BIG_WAVES, BIG_G, false><<<grid, 64 * BIG_WAVES, 0, stream>>>(a);
    }
    int rc = check_launch("act_quant_w4 quant");
    if (rc || !proj_down_t || nb == 1) return rc;
    return lora_sum(workspace, nb, Mp * RANK, lora, stream);
}

// Scratch of wdl_act_quant_w4_static: the quantizer's workspace (column-block partials of the low-rank sums, LN
// statistics) as a file-scope device array, one copy per GPU for the life of the process. Its device address is
// taken once per device with that device current (hipGetSymbolAddress) and kept in scratch_ptr; in host code the
// array's name is not a device address and is never passed to a kernel. Every kernel writes the parts of it that
// a later kernel of the same call reads before that kernel runs (the partials of every column block and row, the
// LayerNorm chunk partials of every row < M), so nothing needs clearing between calls.
static __device__ __align__(256) float scratch[WDL_ACT_QUANT_STATIC_FLOATS];

constexpr int MAX_DEVICES = 64;
float* scratch_ptr[MAX_DEVICES] = {};
std::mutex scratch_lock;

int static_scratch(hipStream_t stream, float** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= MAX_DEVICES)
        return fail(WDL_EHIP, "act_quant_w4_static: no current device");
    if (stream) {
        hipDevice_t sdev = -1;
        if (hipStreamGetDevice(stream, &sdev) != hipSuccess || sdev != dev)
            return fail(WDL_EINVAL, "act_quant_w4_static: the stream belongs to device %d, the current device is %d",
                        int(sdev), dev);
    }
    std::lock_guard<std::mutex> hold(scratch_lock);
    if (!scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || !p)
            return fail(WDL_EHIP, "act_quant_w4_static: hipGetSymbolAddress: %s", hipGetErrorString(e));
        scratch_ptr[dev] = static_cast<float*>(p);
    }
    *out = scratch_ptr[dev];
    return WDL_OK;
}

}  // namespace

extern "C" int wdl_act_quant_w4(const void* x, int64_t ldx, int64_t M, int64_t K, const void* smooth, float qshift,
                                int unsigned_q, const void* proj_down_t, int64_t rank, void* q, void* ascales,
                                float* lora, int64_t Mp, const float* mod_shift, const float* mod_scale,
                                const float* ln_w, const float* ln_b, int ln, float eps, const float* ln_partials,
                                void* v_out, float* workspace, hipStream_t stream) {
    return act_quant_launch(x, ldx, M, K, smooth, qshift, unsigned_q, proj_down_t, rank, q, ascales, lora, Mp,
                            mod_shift, mod_scale, ln_w, ln_b, ln, eps, ln_partials, v_out, workspace, stream);
}

extern "C" int wdl_act_quant_w4_static(const void* x, int64_t ldx, int64_t M, int64_t K, const void* smooth,
                                       float qshift, int unsigned_q, const void* proj_down_t, int64_t rank, void* q,
                                       void* ascales, float* lora, int64_t Mp, const float* mod_shift,
                                       const float* mod_scale, const float* ln_w, const float* ln_b, int ln,
                                       float eps, const float* ln_partials, void* v_out, hipStream_t stream) {
    if (Mp < 0 || K <= 0 || K % 64)
        return fail(WDL_EINVAL, "act_quant_w4_static: bad shape K=%lld Mp=%lld", (long long)K, (long long)Mp);
    const int64_t need = wdl_act_quant_workspace_floats(Mp, K);
    if (need > WDL_ACT_QUANT_STATIC_FLOATS)
        return fail(WDL_EINVAL, "act_quant_w4_static: Mp=%lld K=%lld needs %lld scratch floats, above the static "
                                "maximum of %lld (use wdl_act_quant_w4 with a workspace)", (long long)Mp,
                    (long long)K, (long long)need, (long long)WDL_ACT_QUANT_STATIC_FLOATS);
    float* ws = nullptr;
    const int rc = static_scratch(stream, &ws);
    if (rc) return rc;
    return act_quant_launch(x, ldx, M, K, smooth, qshift, unsigned_q, proj_down_t, rank, q, ascales, lora, Mp,
                            mod_shift, mod_scale, ln_w, ln_b, ln, eps, ln_partials, v_out, ws, stream);
}
