// Shared device helpers and the error channel of the wdl C ABI (gfx950 only).
//
// Every launcher in this library is `extern "C" int wdl_*(...)`: it validates its arguments on the host, launches
// on the caller's stream, never allocates and never synchronises, and returns WDL_OK or an error code with a
// message kept per host thread (wdl_last_error). Floating-point contraction is off for the whole library
// (-ffp-contract=off): every fused multiply-add is written as fmaf, so the rounding of each kernel is the one its
// source shows.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

#define WDL_OK 0
#define WDL_EINVAL 1
#define WDL_EHIP 2

// floats of the static scratch array of wdl_act_quant_w4_static (16 MiB per GPU); the same value as in
// include/wdl.h
#define WDL_ACT_QUANT_STATIC_FLOATS (int64_t(4) << 20)

// element types of strided inputs
#define WDL_F32 0
#define WDL_F16 1
#define WDL_BF16 2
#define WDL_F64 3

namespace wdl {

int fail(int code, const char* fmt, ...);
int check_launch(const char* what);
int cu_count();  // compute units of the current device (cached per device; 0 if the query fails)
// out[i] = sum over b = 0 .. nb-1 (in increasing order) of part[b * n + i], i < n (low-rank partial sums)
int lora_sum(const float* part, int nb, int64_t n, float* out, hipStream_t stream);

// The W4A4 GEMM's operands: fp6 codes, tile-blocked.
//
// Values. Weights w in [-8, 7] are stored as the e3m2 code of 2w (sign, 3 exponent bits of bias 3, 2 mantissa
// bits: every even integer in [-16, 14] is exact); activations q in [-8, 15] as the e2m3 code of q / 2 (bias 1,
// 3 mantissa bits: every multiple of 1/2 in [-4, 7.5] is exact). The matrix cores multiply the two formats at the
// fp6 rate and each product (2w)(q/2) = wq is an exact integer, so a 64-deep group sums to the same integer as the
// int4 dot product.
//
// Bits. Value k (0..63) of a row's 64-deep group goes to half h = k / 32 at position i = k % 32; the 32 codes of
// a half are packed little-endian, code i at bits [6i, 6i + 6) of 24 bytes (four codes in three bytes). This is
// the register layout of v_mfma_f32_32x32x64_f8f6f4 for fp6 operands: lane (row, h) supplies its half's 24 bytes.
//
// Bytes. One row's group is 48 bytes: [half 0 bytes 0..15][half 1 bytes 0..15][half 0 bytes 16..23][half 1 bytes
// 16..23], so a lane reads its 24 bytes as one aligned 16-byte and one aligned 8-byte load. A matrix [R, K]
// (R a multiple of 128, K of 64) is stored as [R / 128][K / 64][128][48]: the group of a 128-row tile that one
// GEMM step reads is one contiguous 6 KB block. The group g of row r starts at blocked6_offset(r, g, K).
constexpr int BLOCK_ROWS = 128;
constexpr int ROW6 = 48;                     // bytes of one row's 64-deep group
constexpr int BLOCK6 = BLOCK_ROWS * ROW6;    // bytes of one 128-row tile's group
__host__ __device__ __forceinline__ int64_t blocked6_offset(int64_t r, int64_t g, int64_t K) {
    return (r / BLOCK_ROWS) * (K / 64) * BLOCK6 + g * BLOCK6 + (r % BLOCK_ROWS) * ROW6;
}
// offset in the 48-byte group row of byte b (0..23) of half h
__host__ __device__ __forceinline__ int half_byte(int h, int b) { return b < 16 ? 16 * h + b : 32 + 8 * h + b - 16; }

// e2m3 code of q / 2 for an integer-valued q with |q| <= 15: |q| 0..3 -> 4|q| (0.5 steps, subnormal up to 1.5),
// 4..7 -> 2|q| + 8, 8..15 -> |q| + 16; the sign in bit 5
__device__ __forceinline__ uint32_t act_code6(float q) {
    const uint32_t m = uint32_t(fabsf(q));
    const uint32_t c = m < 4 ? 4 * m : (m < 8 ? 2 * m + 8 : m + 16);
    return c | (q < 0.0f ? 32u : 0u);
}

// four 6-bit codes in the bytes of x (low first) -> 24 packed bits
__device__ __forceinline__ uint32_t pack4x6(uint32_t x) {
    return (x & 0x3fu) | ((x >> 2) & 0xfc0u) | ((x >> 4) & 0x3f000u) | ((x >> 6) & 0xfc0000u);
}

// ---------------------------------------------------------------- bf16 / fp16 / fp8 conversions (exact, RNE)

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(uint32_t(b) << 16); }

// round to nearest even (gfx950's v_cvt_pk_bf16_f32: identical to the integer RNE recipe on every finite input,
// denormals included, checked bit for bit on the device); NaN stays a NaN
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return __builtin_bit_cast(uint16_t, static_cast<__bf16>(f)); }

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f32_to_f16(float f) { return __half_as_ushort(__float2half_rn(f)); }

// FP8 E4M3FN (OCP): bias 7, no infinities, 0x7f/0xff NaN, largest finite 448, subnormals down to 2^-9.
// Encoding of an fp32 value, rounded to nearest even; magnitudes that round past 448 become NaN (the conversion
// rule of torch.Tensor.to(torch.float8_e4m3fn)).
__device__ __forceinline__ uint8_t f32_to_e4m3(float f);

// Four values as e4m3 bytes (a in the low byte) with the hardware conversion, which equals f32_to_e4m3 on every
// fp32 input of magnitude up to 448 (all 2.28e9 of them checked): quotients x / (max|x| / 448) stay within that
// range up to the last bit of the scale's rounding, which both round to 448.
__device__ __forceinline__ uint32_t e4m3x4(float a, float b, float c, float d) {
    return __builtin_amdgcn_cvt_pk_fp8_f32(c, d, __builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false), true);
}

__device__ __forceinline__ uint8_t f32_to_e4m3(float f) {
    uint32_t u = __float_as_uint(f);
    uint8_t sign = uint8_t((u >> 24) & 0x80u);
    u &= 0x7fffffffu;
    if (u >= 0x43f00000u) return uint8_t(sign | 0x7fu);  // >= 480 or NaN/inf
    if (u < 0x3c800000u) {  // below 2^-6: subnormal, quantum 2^-9
        // a * 512 is exact (a power-of-two scaling of a value far from overflow); rint rounds half to even; a
        // result of 8 is the smallest normal 2^-6, whose encoding is 0x08
        float r = __builtin_rintf(__uint_as_float(u) * 512.0f);
        return uint8_t(sign | uint8_t(r));
    }
    // normal: keep 3 mantissa bits, RNE on the 20 dropped ones
    uint32_t mant_odd = (u >> 20) & 1u;
    u += ((uint32_t)(7 - 127) << 23) + 0x7ffffu + mant_odd;
    return uint8_t(sign | uint8_t(u >> 20));
}

// The IEEE quotient w / d from r = RN(1/d): q0 = RN(w r), e = w - q0 d (exact by fma), q = RN(q0 + e r) -- one
// Markstein correction step, which returns the correctly rounded quotient for binary32 operands away from
// overflow and underflow (checked against IEEE division on every positive bf16 divisor and on 24M random and
// hard-significand fp32 divisors). For w = -0 the correction adds +0 to q0 = -0 and would return +0, so the sign
// is taken from q0 (which always has the quotient's sign). 4 instructions per quotient once the reciprocal of a
// shared divisor is known.
__device__ __forceinline__ float div_rn(float w, float d, float r) {
    const float q0 = w * r;
    const float e = fmaf(-q0, d, w);
    return __builtin_copysignf(fmaf(e, r, q0), q0);
}

// 4 e4m3 codes (bytes of w, low first) to floats with the hardware conversion (exact; e4m3fn as torch decodes it)
__device__ __forceinline__ void e4m3x4_to_f32(uint32_t w, float* f) {
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    const f32x2 lo = __builtin_amdgcn_cvt_pk_f32_fp8(int(w), false), hi = __builtin_amdgcn_cvt_pk_f32_fp8(int(w), true);
    f[0] = lo[0], f[1] = lo[1], f[2] = hi[0], f[3] = hi[1];
}

__device__ __forceinline__ float e4m3_to_f32(uint8_t b) {
    uint32_t sign = uint32_t(b & 0x80u) << 24;
    uint32_t e = (b >> 3) & 0xfu, m = b & 7u;
    if (e == 0xf && m == 7) return __uint_as_float(sign | 0x7fc00000u);
    if (e == 0) {
        float v = float(m) * (1.0f / 512.0f);
        return sign ? -v : v;
    }
    return __uint_as_float(sign | ((e + 120u) << 23) | (m << 20));
}

template <typename T>
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i);

template <>
__device__ __forceinline__ float load_as_f32<float>(const void* p, int64_t i) {
    return static_cast<const float*>(p)[i];
}
template <>
__device__ __forceinline__ float load_as_f32<uint16_t>(const void* p, int64_t i) {  // bf16
    return bf16_to_f32(static_cast<const uint16_t*>(p)[i]);
}
struct half_tag {};
template <>
__device__ __forceinline__ float load_as_f32<half_tag>(const void* p, int64_t i) {
    return f16_to_f32(static_cast<const uint16_t*>(p)[i]);
}

// ---------------------------------------------------------------- wavefront reductions (64 lanes)

// Lane exchanges in registers, not through the LDS crossbar (ds_bpermute, a round trip of the LDS pipeline):
// lane_xor<O> (O = 1, 2, 4, 8) is the value of lane ^ O by DPP within rows of 16 lanes; across rows (O = 16, 32)
// v_permlane16_swap / v_permlane32_swap of a value with itself give each lane its own value and that of lane ^ O,
// in an order that depends on the lane, so they serve commutative combinations only (xor_sum, xor_max: for every
// O the result equals v op (v of lane ^ O), bit for bit).
template <int O>
__device__ __forceinline__ float lane_xor(float v) {
    static_assert(O == 1 || O == 2 || O == 4 || O == 8, "within a row of 16 lanes");
    const int x = __float_as_int(v);
    if constexpr (O == 1) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0xB1, 0xF, 0xF, true));  // [1,0,3,2]
    if constexpr (O == 2) return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x4E, 0xF, 0xF, true));  // [2,3,0,1]
    if constexpr (O == 4)  // half-row mirror (i -> i ^ 7), then quad [3,2,1,0] (i -> i ^ 3)
        return __int_as_float(
            __builtin_amdgcn_mov_dpp(__builtin_amdgcn_mov_dpp(x, 0x141, 0xF, 0xF, true), 0x1B, 0xF, 0xF, true));
    return __int_as_float(__builtin_amdgcn_mov_dpp(x, 0x128, 0xF, 0xF, true));  // row rotate by 8: i -> i ^ 8
}

template <int O>
__device__ __forceinline__ float xor_sum(float v) {
    if constexpr (O == 16 || O == 32) {
        const auto s = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                               : __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return __uint_as_float(s[0]) + __uint_as_float(s[1]);
    } else {
        return v + lane_xor<O>(v);
    }
}

template <int O>
__device__ __forceinline__ float xor_max(float v) {
    if constexpr (O == 16 || O == 32) {
        const auto s = O == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false)
                               : __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
        return fmaxf(__uint_as_float(s[0]), __uint_as_float(s[1]));
    } else {
        return fmaxf(v, lane_xor<O>(v));
    }
}

// butterfly over groups of WIDTH lanes (WIDTH / 2 first, down to 1)
template <int WIDTH>
__device__ __forceinline__ float group_max(float v) {
    if constexpr (WIDTH >= 64) v = xor_max<32>(v);
    if constexpr (WIDTH >= 32) v = xor_max<16>(v);
    if constexpr (WIDTH >= 16) v = xor_max<8>(v);
    if constexpr (WIDTH >= 8) v = xor_max<4>(v);
    if constexpr (WIDTH >= 4) v = xor_max<2>(v);
    if constexpr (WIDTH >= 2) v = xor_max<1>(v);
    return v;
}

template <int WIDTH>
__device__ __forceinline__ float group_sum(float v) {
    if constexpr (WIDTH >= 64) v = xor_sum<32>(v);
    if constexpr (WIDTH >= 32) v = xor_sum<16>(v);
    if constexpr (WIDTH >= 16) v = xor_sum<8>(v);
    if constexpr (WIDTH >= 8) v = xor_sum<4>(v);
    if constexpr (WIDTH >= 4) v = xor_sum<2>(v);
    if constexpr (WIDTH >= 2) v = xor_sum<1>(v);
    return v;
}

}  // namespace wdl
