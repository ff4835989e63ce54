// Sage-2 preparation read straight from the FP8 KV cache and the chunk's own bf16 K/V (kernels/sage_kv.py:28-173).
//
// Token t of a call: t < at comes from the cache (e4m3 value * its fp32 row scale), at <= t < L = at + n from the
// chunk (bf16), t >= L is zero. Three launches:
//   colstats   (grid H x S): per split s of the tokens, partial sums of K and maxima of |V| per (head, channel),
//              each in a fixed order (16 token lanes, then the lanes in order);
//   finalize   (grid H):     k_mean = (sum over splits, in order) / L;  v_scale = max(max |V|, 1e-8) / 2.25;
//              with cached statistics of tokens [0, at) (wdl_sage_cache_stats: their sums and maxima, formed the
//              same way over splits of [0, at)) the splits cover only the chunk's tokens and the sum starts from
//              the cached one;
//   quant_kv   (grid blocks x H): K - mean to int8 with one scale per group g = 0..3 of each 64-token block (tokens
//              8i + 2g, 8i + 2g + 1): scale = max|x| / 127 + 1e-7, q = trunc(x / scale +- 0.5);
//              V / v_scale to e4m3, stored per (head, channel) along the tokens in wdl's order: within a
//              64-token block, position 32 * ((t % 8) / 4) + 4 * (t / 8) + t % 4 holds token t (the key order one
//              lane half of the transposed QK^T MFMA tile produces, so P feeds the PV MFMA unshuffled).
// Layouts: k_int8 [H, Lpad, 128]; k_scale fp32 [H, Lpad / 64 * 4]; v_fp8 [H, 128, Lpad]; Lpad = 64 * ceil(L / 64);
// padding tokens are zero in both.
#include "wdl_common.h"

namespace {

using namespace wdl;

constexpr int D = 128;

struct Src {
    const uint8_t* cache;   // [cap, Hc, D] e4m3
    const float* cscale;    // [cap, Hc]
    const uint16_t* chunk;  // bf16, token stride ld, head stride D
    int64_t ld;
    int64_t Hc, cap;        // heads and rows of the cache
    const int32_t* hmap;    // head h of the call reads cache head hmap[h] (null: h)
    const int32_t* tmap;    // cached token t is cache row tmap[t] (null: t)
};

// cache row index (token row * Hc + head) of cached token t of head h; mapped indices are clamped into the cache
// (the host checks the maps' ranges; the clamp keeps every access inside the buffers whatever they hold)
__device__ __forceinline__ int64_t cache_row(const Src& s, int64_t t, int64_t h) {
    int64_t ct = t, ch = h;
    if (s.tmap) ct = min(max(int64_t(s.tmap[t]), int64_t(0)), s.cap - 1);
    if (s.hmap) ch = min(max(int64_t(s.hmap[h]), int64_t(0)), s.Hc - 1);
    return ct * s.Hc + ch;
}

// 8 channels d0 .. d0 + 7 of token t (head h) as floats: cached tokens from e4m3 times their row scale, chunk
// tokens from bf16, tokens >= L zero. CACHE / CHUNK: the caller knows the token's source (uniform paths).
enum { MIXED = 0, CACHE = 1, CHUNK = 2 };
template <int SRC>
__device__ __forceinline__ void load_token8(const Src& s, int64_t t, int64_t h, int64_t H, int64_t at, int64_t L,
                                            int d0, float* f) {
    if (SRC == CACHE || (SRC == MIXED && t < at)) {
        const int64_t row = cache_row(s, t, h);
        const uint2 raw = *reinterpret_cast<const uint2*>(s.cache + row * D + d0);
        const float sc = s.cscale[row];
        e4m3x4_to_f32(raw.x, f);
        e4m3x4_to_f32(raw.y, f + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = f[j] * sc;
    } else if (SRC == CHUNK || t < L) {
        const uint4 raw = *reinterpret_cast<const uint4*>(s.chunk + (t - at) * s.ld + h * D + d0);
        const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            f[2 * j] = __uint_as_float(w[j] << 16);
            f[2 * j + 1] = __uint_as_float(w[j] & 0xffff0000u);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 8; ++j) f[j] = 0.0f;
    }
}

constexpr int UNROLL = 4;  // tokens per lane in flight in the statistics pass

// tokens lo, lo + 16, ... < hi of one source: the K sums and |V| maxima of this lane's 8 channels, loads of UNROLL
// tokens issued before they are used
template <int SRC>
__device__ __forceinline__ void colstats_range(const Src& k, const Src& v, int64_t h, int64_t H, int64_t at,
                                               int64_t L, int64_t lo, int64_t hi, int d0, float* ks, float* vm) {
    int64_t tok = lo;
    for (; tok + 16 * (UNROLL - 1) < hi; tok += 16 * UNROLL) {
        float fk[UNROLL][8], fv[UNROLL][8];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            load_token8<SRC>(k, tok + 16 * u, h, H, at, L, d0, fk[u]);
            load_token8<SRC>(v, tok + 16 * u, h, H, at, L, d0, fv[u]);
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                ks[j] = ks[j] + fk[u][j];
                vm[j] = fmaxf(vm[j], fabsf(fv[u][j]));
            }
    }
    for (; tok < hi; tok += 16) {
        float f[8];
        load_token8<SRC>(k, tok, h, H, at, L, d0, f);
#pragma unroll
        for (int j = 0; j < 8; ++j) ks[j] = ks[j] + f[j];
        load_token8<SRC>(v, tok, h, H, at, L, d0, f);
#pragma unroll
        for (int j = 0; j < 8; ++j) vm[j] = fmaxf(vm[j], fabsf(f[j]));
    }
}

// the tokens [t0, L) in S splits
__global__ __launch_bounds__(256) void colstats_kernel(Src k, Src v, int64_t H, int64_t at, int64_t t0, int64_t L,
                                                       int S, float* part_k, float* part_v) {
    __shared__ float red[2][16][D];
    const int64_t h = blockIdx.x, s = blockIdx.y;
    const int t = threadIdx.x, lane_tok = t / 16, d0 = (t % 16) * 8;
    const int64_t per = (L - t0 + S - 1) / S;
    const int64_t lo = t0 + s * per, hi = min(L, lo + per);
    float ks[8] = {}, vm[8] = {};
    // this lane's tokens lo + lane_tok + 16 i: the cached ones first, then the chunk's
    const int64_t first = lo + lane_tok;
    const int64_t split = first >= at ? first : first + (at - first + 15) / 16 * 16;  // first chunk token
    colstats_range<CACHE>(k, v, h, H, at, L, first, min(hi, split), d0, ks, vm);
    colstats_range<CHUNK>(k, v, h, H, at, L, max(first, split), hi, d0, ks, vm);
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        red[0][lane_tok][d0 + j] = ks[j];
        red[1][lane_tok][d0 + j] = vm[j];
    }
    __syncthreads();
    if (t < D) {
        float a = 0.0f, m = 0.0f;
        for (int i = 0; i < 16; ++i) {
            a = a + red[0][i][t];
            m = fmaxf(m, red[1][i][t]);
        }
        part_k[(s * H + h) * D + t] = a;
        part_v[(s * H + h) * D + t] = m;
    }
}

// base: null, or cached statistics [2][H][D] (K sums, |V| maxima) the splits' values are added to; raw: write the
// sums and maxima into k_mean (as [2][H][D]) instead of the mean and v_scale
__global__ void finalize_kernel(const float* part_k, const float* part_v, int S, int64_t H, int64_t L, float* k_mean,
                                float* v_scale, const float* base, int raw) {
    const int64_t h = blockIdx.x;
    const int d = threadIdx.x;
    // the splits in increasing order; the loads of a batch of 16 are all issued before the first add (one memory
    // round trip per batch, not one per split)
    constexpr int BATCH = 16;
    float a = base ? base[h * D + d] : 0.0f, m = base ? base[(H + h) * D + d] : 0.0f;
    for (int s0 = 0; s0 < S; s0 += BATCH) {
        float pk[BATCH], pv[BATCH];
#pragma unroll
        for (int j = 0; j < BATCH; ++j) {
            const bool in = s0 + j < S;
            pk[j] = in ? part_k[((s0 + j) * H + h) * D + d] : 0.0f;
            pv[j] = in ? part_v[((s0 + j) * H + h) * D + d] : 0.0f;
        }
#pragma unroll
        for (int j = 0; j < BATCH; ++j)
            if (s0 + j < S) {
                a = a + pk[j];
                m = fmaxf(m, pv[j]);
            }
    }
    if (raw) {
        k_mean[h * D + d] = a;
        k_mean[(H + h) * D + d] = m;
        return;
    }
    k_mean[h * D + d] = a / float(L);
    v_scale[h * D + d] = fmaxf(m, 1e-8f) / 2.25f;
}

__device__ __forceinline__ int v_position(int t) { return 32 * ((t % 8) / 4) + 4 * (t / 8) + t % 4; }

// 32 e4m3 values (channels d0 .. d0 + 31, 32 contiguous bytes) of cached token t times the row's scale: two 16-byte
// loads and one scale load (the values and products of four load_token8<CACHE> calls)
__device__ __forceinline__ void load_cached32(const Src& s, int64_t t, int64_t h, int64_t H, int d0,
                                              float (&f)[4][8]) {
    const int64_t row = cache_row(s, t, h);
    const uint4* src = reinterpret_cast<const uint4*>(s.cache + row * D + d0);
    const uint4 r0 = src[0], r1 = src[1];
    const float sc = s.cscale[row];
    const uint32_t w[8] = {r0.x, r0.y, r0.z, r0.w, r1.x, r1.y, r1.z, r1.w};
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        e4m3x4_to_f32(w[2 * c], f[c]);
        e4m3x4_to_f32(w[2 * c + 1], f[c] + 4);
#pragma unroll
        for (int j = 0; j < 8; ++j) f[c][j] = f[c][j] * sc;
    }
}

template <int SRC>
__device__ __forceinline__ void quant_block(const Src& k, const Src& v, int64_t h, int64_t H, int64_t at, int64_t L,
                                            int64_t tok, int dq, float (&fk)[4][8], float (&fv)[4][8]) {
    if (SRC == CACHE) {
        load_cached32(k, tok, h, H, dq, fk);
        load_cached32(v, tok, h, H, dq, fv);
        return;
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        load_token8<SRC>(k, tok, h, H, at, L, dq + c * 8, fk[c]);
        load_token8<SRC>(v, tok, h, H, at, L, dq + c * 8, fv[c]);
    }
}

// Row `row` of an FP8 cache from 32 channels (dq .. dq + 31) per thread, the 4 threads of a token in consecutive
// lanes: the arithmetic of wdl_kv_append_fp8 (kv_cache.hip), scale = max(max |x| over the 128 channels, 1e-12) /
// 448, codes e4m3 of the IEEE quotients x / scale (div_rn on the reciprocal), so the bytes and scales are the
// same (the hardware conversion, e4m3x4). Every thread takes part in the row maximum; only `on` threads store.
__device__ __forceinline__ void append_row(const float (&f)[4][8], uint8_t* cache, float* scales, int64_t row, int dq,
                                           bool on) {
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) amax = fmaxf(amax, fabsf(f[c][j]));
    amax = xor_max<2>(xor_max<1>(amax));  // the token's 4 threads
    const float scale = fmaxf(amax, 1e-12f) / 448.0f;
    if (!on) return;
    const float rs = 1.0f / scale;
    uint32_t w[8];
#pragma unroll
    for (int b = 0; b < 8; ++b) {
        const float* x = f[b / 2] + 4 * (b % 2);
        w[b] = e4m3x4(div_rn(x[0], scale, rs), div_rn(x[1], scale, rs), div_rn(x[2], scale, rs),
                      div_rn(x[3], scale, rs));
    }
    uint4* dst = reinterpret_cast<uint4*>(cache + row * D + dq);
    dst[0] = make_uint4(w[0], w[1], w[2], w[3]);
    dst[1] = make_uint4(w[4], w[5], w[6], w[7]);
    if (dq == 0) scales[row] = scale;
}

// Where the chunk's rows also go into the FP8 caches (Append::k non-null): rows token * H + head, unmapped caches.
struct Append {
    uint8_t* k;
    float* ks;
    uint8_t* v;
    float* vs;
};

__global__ __launch_bounds__(256) void quant_kv_kernel(Src k, Src v, int64_t H, int64_t at, int64_t L, int64_t Lpad,
                                                       const float* k_mean, const float* v_scale, int8_t* k_out,
                                                       float* k_scale, uint8_t* v_out, Append app) {
    __shared__ float gmax[64][4];
    __shared__ __attribute__((aligned(16))) uint8_t vt[D][64 + 4];  // codes [channel][position], 4-byte rows
    __shared__ __attribute__((aligned(16))) float stat[3][D];  // k_mean, v_scale, 1 / v_scale of the head
    const int64_t blk = blockIdx.x, h = blockIdx.y;
    const int t = threadIdx.x, tt = t / 4, dq = (t % 4) * 32;
    const int64_t tok = blk * 64 + tt;
    if (t < D) {
        stat[0][t] = k_mean[h * D + t];
        const float vs = v_scale[h * D + t];
        stat[1][t] = vs;
        stat[2][t] = 1.0f / vs;
    }
    // all loads of this thread's token first (the block's source is uniform unless it straddles at or L)
    float fk[4][8], fv[4][8];
    const int64_t b0 = blk * 64, b1 = b0 + 64;
    if (b1 <= at) quant_block<CACHE>(k, v, h, H, at, L, tok, dq, fk, fv);
    else if (b0 >= at && b1 <= L) quant_block<CHUNK>(k, v, h, H, at, L, tok, dq, fk, fv);
    else quant_block<MIXED>(k, v, h, H, at, L, tok, dq, fk, fv);
    if (app.k && b1 > at) {  // the block holds chunk tokens (uniform)
        const bool on = tok >= at && tok < L;
        append_row(fk, app.k, app.ks, tok * H + h, dq, on);
        append_row(fv, app.v, app.vs, tok * H + h, dq, on);
    }
    __syncthreads();
    // K - mean: 32 channels of one token per thread. Tokens >= L loaded as +0 (load_token8), so with live = 0 the
    // fma gives +0 and with live = 1 it is the one rounding of fk - mean; their V quotients are +0, code 0.
    const float live = tok < L ? 1.0f : 0.0f;
    float x[32];
    float amax = 0.0f;
#pragma unroll
    for (int c = 0; c < 4; ++c)
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            const float y = fmaf(-stat[0][dq + c * 8 + j], live, fk[c][j]);
            x[c * 8 + j] = y;
            amax = fmaxf(amax, fabsf(y));
        }
    gmax[tt][t % 4] = amax;
    // V codes into the transposed tile (V / v_scale is below 2.25 in magnitude: the conversion never saturates).
    // A dword holds 4 channels of the thread's token; a 4 x 4 byte transpose between the 4 lanes that hold tokens
    // 4k .. 4k + 3 of the same channel quarter (lanes 4 apart in a row of 16: DPP, then v_perm) leaves each lane 4
    // consecutive positions of one channel (v_position keeps 4 consecutive tokens at consecutive positions), so
    // one 4-byte LDS store replaces four byte stores.
    {
        const int ti = tt % 4;  // the token's place in its group of 4; the lane ends with channel d + ti
        const uint32_t sel1 = (ti & 2) ? 0x03020706u : 0x05040100u;  // exchange halves with the token ti ^ 2
        const uint32_t sel2 = (ti & 1) ? 0x03070105u : 0x06020400u;  // exchange bytes with the token ti ^ 1
        const int pos = v_position(tt - ti);
#pragma unroll
        for (int c4 = 0; c4 < 8; ++c4) {
            const int d = dq + 4 * c4, c = c4 / 2, j = 4 * (c4 % 2);
            float y[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) y[e] = div_rn(fv[c][j + e], stat[1][d + e], stat[2][d + e]);
            uint32_t w = __builtin_amdgcn_cvt_pk_fp8_f32(y[0], y[1], 0, false);
            w = __builtin_amdgcn_cvt_pk_fp8_f32(y[2], y[3], w, true);
            w = __builtin_amdgcn_perm(__float_as_uint(lane_xor<8>(__uint_as_float(w))), w, sel1);
            w = __builtin_amdgcn_perm(__float_as_uint(lane_xor<4>(__uint_as_float(w))), w, sel2);
            *reinterpret_cast<uint32_t*>(&vt[d + ti][pos]) = w;
        }
    }
    __syncthreads();
    const int g = (tt % 8) / 2;
    float m = 0.0f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
#pragma unroll
        for (int p = 0; p < 2; ++p) {
            const int member = 8 * i + 2 * g + p;
#pragma unroll
            for (int q = 0; q < 4; ++q) m = fmaxf(m, gmax[member][q]);
        }
    }
    const float scale = m / 127.0f + 1e-7f;
    const float rscale = 1.0f / scale;
    if (t % 4 == 0 && (tt % 8) == 2 * g && tt < 8) k_scale[h * (Lpad / 64 * 4) + blk * 4 + g] = scale;
    int8_t* kd = k_out + (h * Lpad + tok) * D + dq;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            uint32_t word = 0;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                // the correctly rounded quotient (div_rn without its sign fix: a zero of either sign rounds to 0),
                // rounded half away from zero; r + 128 is an integer in [1, 255], packed as an exact u8 conversion
                // and turned into the two's-complement byte by the xor below
                const float xv = x[c * 16 + b * 4 + e];
                const float q0 = xv * rscale;
                const float y = fmaf(fmaf(-q0, scale, xv), rscale, q0);
                const float r = __builtin_truncf(y + __builtin_copysignf(0.5f, y)) + 128.0f;
                word = __builtin_amdgcn_cvt_pk_u8_f32(r, e, word);
            }
            w[b] = word ^ 0x80808080u;
        }
        *reinterpret_cast<uint4*>(kd + c * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
    // V: thread -> channel t / 2, 32 positions
    const int d = t / 2, p0 = (t % 2) * 32;
    uint8_t* vd = v_out + (h * D + d) * Lpad + blk * 64 + p0;
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        uint32_t w[4];
#pragma unroll
        for (int b = 0; b < 4; ++b) w[b] = *reinterpret_cast<const uint32_t*>(&vt[d][p0 + c * 16 + b * 4]);
        *reinterpret_cast<uint4*>(vd + c * 16) = make_uint4(w[0], w[1], w[2], w[3]);
    }
}

// ---------------------------------------------------------------- the reference's Sage operand layouts
// live::sage_sm89 (native/ops/sage_ops.cpp:12-19) takes the operands kernels/sage_kv.py:141-176 builds: int8 K
// [L, H, 128] (token-major, heads interleaved) and fp8 V [128, H, Lpad] whose 16-token groups are stored in Sage's
// order (token j of a group at 4 (p % 4) + 2 (p / 4) + j % 2, p = j / 2; sage_kv.py:101-103). The scales have
// wdl's layouts already (q_scale [H, blocks * 8], k_scale [H, Lpad / 64 * 4], v_scale [H, 128]).

// K: one thread per 16 bytes of the output [H, Lpad, 128]; tokens L .. Lpad - 1 zero.
__global__ __launch_bounds__(256) void sm89_k_kernel(const int8_t* __restrict__ k, int64_t ldk, int64_t H,
                                                    int64_t L, int64_t Lpad, int8_t* __restrict__ out) {
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;  // 16-byte chunk of the output
    if (i >= H * Lpad * 8) return;
    const int64_t c = i % 8, t = (i / 8) % Lpad, h = i / (8 * Lpad);
    uint4 v = make_uint4(0, 0, 0, 0);
    if (t < L) v = *reinterpret_cast<const uint4*>(k + t * ldk + h * D + c * 16);
    *reinterpret_cast<uint4*>(out + (h * Lpad + t) * D + c * 16) = v;
}

// position of token j (0..15) of a 16-token group in Sage's order
__device__ __forceinline__ int sage16_pos(int j) {
    const int p = j / 2;
    return (p % 4) * 4 + (p / 4) * 2 + j % 2;
}

// V: one thread per (head, channel, 64-token block): the block's 64 bytes in Sage's order in, wdl's order out
// (output position 32 a + 4 b + c holds token 8 b + 4 a + c).
__global__ __launch_bounds__(256) void sm89_v_kernel(const uint8_t* __restrict__ v, int64_t sd, int64_t sh,
                                                    int64_t H, int64_t Lpad, uint8_t* __restrict__ out) {
    const int64_t nb = Lpad / 64;
    const int64_t i = int64_t(blockIdx.x) * 256 + threadIdx.x;
    if (i >= H * D * nb) return;
    const int64_t blk = i % nb, d = (i / nb) % D, h = i / (nb * D);
    const uint8_t* src = v + d * sd + h * sh + blk * 64;
    uint32_t in[16];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
        const uint4 w = *reinterpret_cast<const uint4*>(src + 16 * c);
        in[4 * c] = w.x, in[4 * c + 1] = w.y, in[4 * c + 2] = w.z, in[4 * c + 3] = w.w;
    }
    uint32_t o[16];
#pragma unroll
    for (int q = 0; q < 16; ++q) {
        uint32_t word = 0;
#pragma unroll
        for (int b = 0; b < 4; ++b) {
            const int pos = 4 * q + b;                                     // output position in the block
            const int t = 8 * ((pos % 32) / 4) + 4 * (pos / 32) + pos % 4;  // its token
            const int s = (t & ~15) + sage16_pos(t & 15);                   // where Sage's order keeps it
            word |= ((in[s / 4] >> (8 * (s % 4))) & 0xffu) << (8 * b);
        }
        o[q] = word;
    }
    uint8_t* dst = out + (h * D + d) * Lpad + blk * 64;
#pragma unroll
    for (int c = 0; c < 4; ++c)
        *reinterpret_cast<uint4*>(dst + 16 * c) = make_uint4(o[4 * c], o[4 * c + 1], o[4 * c + 2], o[4 * c + 3]);
}

}  // namespace

// workspace floats: 2 * S * H * 128 (partials) + 2 * H * 128 (k_mean, v_scale)
extern "C" int64_t wdl_sage_prep_workspace_floats(int64_t heads, int splits) { return (2 * splits + 2) * heads * D; }

static int sage_prep_launch(const void* cache_k, const float* cache_ks, const void* cache_v, const float* cache_vs,
                            int64_t capacity, int64_t cache_heads, const int32_t* heads_map,
                            const int32_t* tokens_map, const void* k, int64_t ldk, const void* v, int64_t ldv,
                            int64_t heads, int64_t at, int64_t n, int splits, float* workspace, void* k_int8,
                            float* k_scale, void* v_fp8, float* k_mean_out, float* v_scale_out, hipStream_t stream,
                            const float* cache_stats = nullptr, Append app = Append{}) {
    const int64_t L = at + n;
    if (at < 0 || n < 0 || heads <= 0 || at > capacity || splits < 1 || ldk < heads * D || ldv < heads * D ||
        cache_heads < heads || (!heads_map && cache_heads != heads))
        return fail(WDL_EINVAL, "sage_prep: bad shape");
    if (!cache_k || !cache_ks || !cache_v || !cache_vs || !k || !v || !workspace || !k_int8 || !k_scale || !v_fp8)
        return fail(WDL_EINVAL, "sage_prep: null pointer");
    if ((reinterpret_cast<uintptr_t>(k) | reinterpret_cast<uintptr_t>(v) | (ldk * 2) | (ldv * 2)) % 16)
        return fail(WDL_EINVAL, "sage_prep: chunk rows must be 16-byte aligned");
    if ((reinterpret_cast<uintptr_t>(cache_k) | reinterpret_cast<uintptr_t>(cache_v)) % 16)
        return fail(WDL_EINVAL, "sage_prep: the caches must be 16-byte aligned");
    if (L == 0) return WDL_OK;
    if (capacity < 1) return fail(WDL_EINVAL, "sage_prep: empty cache");
    const int64_t Lpad = (L + 63) / 64 * 64;
    Src sk{static_cast<const uint8_t*>(cache_k), cache_ks, static_cast<const uint16_t*>(k), ldk, cache_heads,
           capacity, heads_map, tokens_map};
    Src sv{static_cast<const uint8_t*>(cache_v), cache_vs, static_cast<const uint16_t*>(v), ldv, cache_heads,
           capacity, heads_map, tokens_map};
    float* part_k = workspace;
    float* part_v = workspace + int64_t(splits) * heads * D;
    float* k_mean = k_mean_out ? k_mean_out : workspace + 2 * int64_t(splits) * heads * D;
    float* v_scale = v_scale_out ? v_scale_out : k_mean + heads * D;
    // with cached statistics of tokens [0, at), only the chunk's tokens are summed here
    const int64_t t0 = cache_stats ? at : 0;
    colstats_kernel<<<dim3(unsigned(heads), unsigned(splits)), 256, 0, stream>>>(sk, sv, heads, at, t0, L, splits,
                                                                                 part_k, part_v);
    int rc = check_launch("sage_prep colstats");
    if (rc) return rc;
    finalize_kernel<<<unsigned(heads), D, 0, stream>>>(part_k, part_v, splits, heads, L, k_mean, v_scale, cache_stats,
                                                       0);
    rc = check_launch("sage_prep finalize");
    if (rc) return rc;
    quant_kv_kernel<<<dim3(unsigned(Lpad / 64), unsigned(heads)), 256, 0, stream>>>(
        sk, sv, heads, at, L, Lpad, k_mean, v_scale, static_cast<int8_t*>(k_int8), k_scale,
        static_cast<uint8_t*>(v_fp8), app);
    return check_launch("sage_prep quant_kv");
}

extern "C" int wdl_sage_prep(const void* cache_k, const float* cache_ks, const void* cache_v, const float* cache_vs,
                             int64_t capacity, const void* k, int64_t ldk, const void* v, int64_t ldv, int64_t heads,
                             int64_t at, int64_t n, int splits, float* workspace, void* k_int8, float* k_scale,
                             void* v_fp8, float* k_mean_out, float* v_scale_out, hipStream_t stream) {
    return sage_prep_launch(cache_k, cache_ks, cache_v, cache_vs, capacity, heads, nullptr, nullptr, k, ldk, v, ldv,
                            heads, at, n, splits, workspace, k_int8, k_scale, v_fp8, k_mean_out, v_scale_out, stream);
}

extern "C" int wdl_sage_prep_mapped(const void* cache_k, const float* cache_ks, const void* cache_v,
                                    const float* cache_vs, int64_t capacity, int64_t cache_heads,
                                    const int32_t* heads_map, const int32_t* tokens_map, const void* k, int64_t ldk,
                                    const void* v, int64_t ldv, int64_t heads, int64_t at, int64_t n, int splits,
                                    float* workspace, void* k_int8, float* k_scale, void* v_fp8, float* k_mean_out,
                                    float* v_scale_out, hipStream_t stream) {
    return sage_prep_launch(cache_k, cache_ks, cache_v, cache_vs, capacity, cache_heads, heads_map, tokens_map, k,
                            ldk, v, ldv, heads, at, n, splits, workspace, k_int8, k_scale, v_fp8, k_mean_out,
                            v_scale_out, stream);
}

extern "C" int wdl_sage_cache_stats(const void* cache_k, const float* cache_ks, const void* cache_v,
                                    const float* cache_vs, int64_t capacity, int64_t heads, int64_t at, int splits,
                                    float* workspace, float* stats, hipStream_t stream) {
    if (at < 0 || heads <= 0 || at > capacity || capacity < 1 || splits < 1)
        return fail(WDL_EINVAL, "sage_cache_stats: bad shape");
    if (!cache_k || !cache_ks || !cache_v || !cache_vs || !workspace || !stats)
        return fail(WDL_EINVAL, "sage_cache_stats: null pointer");
    if ((reinterpret_cast<uintptr_t>(cache_k) | reinterpret_cast<uintptr_t>(cache_v)) % 16)
        return fail(WDL_EINVAL, "sage_cache_stats: the caches must be 16-byte aligned");
    // tokens [0, at), all from the cache (no chunk: the chunk source is never read)
    Src sk{static_cast<const uint8_t*>(cache_k), cache_ks, nullptr, heads * D, heads, capacity, nullptr, nullptr};
    Src sv{static_cast<const uint8_t*>(cache_v), cache_vs, nullptr, heads * D, heads, capacity, nullptr, nullptr};
    float* part_k = workspace;
    float* part_v = workspace + int64_t(splits) * heads * D;
    colstats_kernel<<<dim3(unsigned(heads), unsigned(splits)), 256, 0, stream>>>(sk, sv, heads, at, 0, at, splits,
                                                                                 part_k, part_v);
    const int rc = check_launch("sage_cache_stats colstats");
    if (rc) return rc;
    finalize_kernel<<<unsigned(heads), D, 0, stream>>>(part_k, part_v, splits, heads, at, stats, nullptr, nullptr, 1);
    return check_launch("sage_cache_stats finalize");
}

extern "C" int wdl_sage_prep_cached(const void* cache_k, const float* cache_ks, const void* cache_v,
                                    const float* cache_vs, int64_t capacity, const void* k, int64_t ldk,
                                    const void* v, int64_t ldv, int64_t heads, int64_t at, int64_t n,
                                    const float* cache_stats, int splits, float* workspace, void* k_int8,
                                    float* k_scale, void* v_fp8, float* k_mean_out, float* v_scale_out,
                                    hipStream_t stream) {
    if (!cache_stats) return fail(WDL_EINVAL, "sage_prep_cached: null cache statistics");
    return sage_prep_launch(cache_k, cache_ks, cache_v, cache_vs, capacity, heads, nullptr, nullptr, k, ldk, v, ldv,
                            heads, at, n, splits, workspace, k_int8, k_scale, v_fp8, k_mean_out, v_scale_out, stream,
                            cache_stats);
}

extern "C" int wdl_sage_prep_cached_append(void* cache_k, float* cache_ks, void* cache_v, float* cache_vs,
                                           int64_t capacity, const void* k, int64_t ldk, const void* v, int64_t ldv,
                                           int64_t heads, int64_t at, int64_t n, const float* cache_stats, int splits,
                                           float* workspace, void* k_int8, float* k_scale, void* v_fp8,
                                           float* k_mean_out, float* v_scale_out, hipStream_t stream) {
    if (!cache_stats) return fail(WDL_EINVAL, "sage_prep_cached_append: null cache statistics");
    if (at < 0 || n < 0 || at + n > capacity)
        return fail(WDL_EINVAL, "sage_prep_cached_append: rows %lld .. %lld outside the cache of %lld", (long long)at,
                    (long long)(at + n), (long long)capacity);
    return sage_prep_launch(cache_k, cache_ks, cache_v, cache_vs, capacity, heads, nullptr, nullptr, k, ldk, v, ldv,
                            heads, at, n, splits, workspace, k_int8, k_scale, v_fp8, k_mean_out, v_scale_out, stream,
                            cache_stats,
                            Append{static_cast<uint8_t*>(cache_k), cache_ks, static_cast<uint8_t*>(cache_v), cache_vs});
}

extern "C" int wdl_sage_sm89_relayout(const void* k_i8, int64_t ldk, const void* v_fp8, int64_t v_stride_d,
                                      int64_t v_stride_h, int64_t L, int64_t heads, void* k_out, void* v_out,
                                      hipStream_t stream) {
    if (L <= 0 || heads <= 0 || ldk < heads * D || v_stride_h < (L + 63) / 64 * 64 || v_stride_d < heads * v_stride_h)
        return fail(WDL_EINVAL, "sage_sm89_relayout: bad shape");
    if (!k_i8 || !v_fp8 || !k_out || !v_out) return fail(WDL_EINVAL, "sage_sm89_relayout: null pointer");
    if ((reinterpret_cast<uintptr_t>(k_i8) | reinterpret_cast<uintptr_t>(v_fp8) | reinterpret_cast<uintptr_t>(k_out) |
         reinterpret_cast<uintptr_t>(v_out) | ldk | v_stride_d | v_stride_h) % 16)
        return fail(WDL_EINVAL, "sage_sm89_relayout: buffers and strides must be 16-byte aligned");
    const int64_t Lpad = (L + 63) / 64 * 64;
    const int64_t nk = heads * Lpad * 8, nv = heads * D * (Lpad / 64);
    sm89_k_kernel<<<unsigned((nk + 255) / 256), 256, 0, stream>>>(static_cast<const int8_t*>(k_i8), ldk, heads, L,
                                                                  Lpad, static_cast<int8_t*>(k_out));
    const int rc = check_launch("sage_sm89_relayout k");
    if (rc) return rc;
    sm89_v_kernel<<<unsigned((nv + 255) / 256), 256, 0, stream>>>(static_cast<const uint8_t*>(v_fp8), v_stride_d,
                                                                  v_stride_h, heads, Lpad,
                                                                  static_cast<uint8_t*>(v_out));
    return check_launch("sage_sm89_relayout v");
}
