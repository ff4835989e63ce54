/* wdl — MI355X (gfx950) C ABI of the quantized Wan DiT block hot path (lib/libwdl.so).
 *
 * Conventions for every entry point:
 *  - plain device pointers, int64 sizes and element strides, and the caller's hipStream_t (passed as void*);
 *  - the caller owns and allocates every buffer (outputs and workspaces); nothing here allocates, frees or
 *    synchronises, so every call can be captured into a HIP graph;
 *  - the return value is WDL_OK (0) or an error code; wdl_last_error() gives the message of the last failure on
 *    the calling host thread. Arguments are validated before any launch: a failure writes nothing.
 *
 * Element type codes for strided floating inputs: 0 = fp32, 1 = fp16, 2 = bf16, 3 = fp64.
 * fp8 means E4M3FN (OCP), stored as bytes; bf16 is stored as uint16.
 */
#ifndef WDL_H
#define WDL_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define WDL_OK 0
#define WDL_EINVAL 1
#define WDL_EHIP 2

typedef void* wdl_stream_t; /* a hipStream_t */

/* Message of the last failed call on this host thread ("" after a success). */
const char* wdl_last_error(void);
int wdl_abi_version(void);

/* FP8 KV-cache append. Replaces store_kv_fp8 / wan_dit_lab::store_kv_fp8_<hash>
 * (src/wan_dit_lab/kernels/cache_fp8.py:59-72, 75-105) and KVCache.store's fp8 branch
 * (src/wan_dit_lab/generation/causal.py:177-181).
 * k, v: [B, n, H, D] of element type k_dtype / v_dtype with element strides k_strides[4] / v_strides[4];
 * cache_k, cache_v: fp8 [B, capacity, H, D] contiguous; cache_ks, cache_vs: fp32 [B, capacity, H, 1].
 * Rows (b, t, h) go to cache token at + t: scale = max(max|x|, 1e-12) / 448, value = e4m3(x / scale). */
int wdl_kv_append_fp8(const void* k, int k_dtype, const int64_t* k_strides, const void* v, int v_dtype,
                      const int64_t* v_strides, int64_t B, int64_t n, int64_t H, int64_t D, void* cache_k,
                      float* cache_ks, void* cache_v, float* cache_vs, int64_t capacity, int64_t at,
                      wdl_stream_t stream);

/* Workspace (in floats) that wdl_act_quant_w4 needs for Mp padded rows of K values. */
int64_t wdl_act_quant_workspace_floats(int64_t Mp, int64_t K);

/* W4A4 activation quantizer (+ low-rank down projection, + optional fused LayerNorm and adaLN modulation).
 * Replaces Nunchaku's quantize_w4a4_act_fuse_lora behind live::w4a4_linear (native/ops/w4a4_ops.cpp:17-29; the
 * quantizer itself is absent from the reference tree) and the norm/modulation of WanBlock.forward
 * (src/wan_dit_lab/models/block.py:25,28; models/layer_norm.py:4-7).
 * x: bf16 [M, K], row stride ldx (16-byte aligned rows); smooth: bf16 [K]; proj_down_t: bf16 [32, K] or NULL.
 * v = x, or with ln != 0: v = bf16(LN(x)[*ln_w + ln_b] * (1 + mod_scale) + mod_shift) (fp32 vectors, NULL = absent).
 * u = (v + qshift) / smooth; per row and 64-group: scale = bf16(max|u| / qmax) (qmax 7, or 15 if unsigned_q),
 * q = clamp(rint(u / scale)). Outputs: q as fp6 codes of the integers [Mp, K] in the operand format (below);
 * ascales bf16 [K/64, Mp]; lora fp32 [Mp, 32] = v . proj_down; rows M..Mp-1 zero. Mp % 128 == 0. v_out (bf16
 * [M, K]) optional copy of v.
 * LayerNorm statistics (K <= 4096) from chunk partials of x: ln_partials fp32 [M][K / 32][2] (16-byte aligned) as
 * the residual epilogue of wdl_w4a4_gemm writes them for the rows it produces, or NULL (then the call forms them
 * from x first, one more launch). Per row and 32-value chunk: (S, M2) = the chunk's sum and its sum of squared
 * deviations from S / 32, each as 8 quads of 4 values summed in order, the quads combined as
 * ((t0 + t1) + (t2 + t3)) + ((t4 + t5) + (t6 + t7)); the row's C chunks merged by 8 slots (slot j: the chunk
 * pairs j, j + 8, ... = chunks 2p, 2p + 1, in chunk order from +0, the slots combined as the same tree): mean =
 * sum S / K, M2 = sum of
 * M2_c + 32 (S_c / 32 - mean)^2, rstd = 1 / sqrt(M2 / K + eps) (the oracle's order).
 * workspace: wdl_act_quant_workspace_floats(Mp, K). */
int wdl_act_quant_w4(const void* x, int64_t ldx, int64_t M, int64_t K, const void* smooth, float qshift,
                     int unsigned_q, const void* proj_down_t, int64_t rank, void* q, void* ascales, float* lora,
                     int64_t Mp, const float* mod_shift, const float* mod_scale, const float* ln_w,
                     const float* ln_b, int ln, float eps, const float* ln_partials, void* v_out, float* workspace,
                     wdl_stream_t stream);

/* wdl_act_quant_w4 without the workspace argument, for callers that cannot allocate device memory (code under HIP
 * graph capture that must not allocate, tight serving loops, harnesses that forbid hipMalloc). No counterpart in the
 * reference. The scratch is a static device array of WDL_ACT_QUANT_STATIC_FLOATS floats (16 MiB) per GPU, held
 * until the process ends; a shape with wdl_act_quant_workspace_floats(Mp, K) above that is rejected (WDL_EINVAL)
 * before any launch (Mp <= 4608 at K = 14336, Mp <= 7168 at K = 3072). Nothing is allocated or freed. The first
 * call on a device looks up that device's copy of the array; the stream must belong to the current device. All
 * calls on one GPU share its array: calls that overlap in time on one GPU (different streams, or threads) race,
 * as calls sharing one workspace of wdl_act_quant_w4 do. Outputs are bit-identical to wdl_act_quant_w4's. */
#define WDL_ACT_QUANT_STATIC_FLOATS ((int64_t)4 << 20)
int wdl_act_quant_w4_static(const void* x, int64_t ldx, int64_t M, int64_t K, const void* smooth, float qshift,
                            int unsigned_q, const void* proj_down_t, int64_t rank, void* q, void* ascales,
                            float* lora, int64_t Mp, const float* mod_shift, const float* mod_scale,
                            const float* ln_w, const float* ln_b, int ln, float eps, const float* ln_partials,
                            void* v_out, wdl_stream_t stream);

/* Operand format of the W4A4 GEMM (both sides; R % 128 == 0, K % 64 == 0), R * K * 3/4 bytes:
 * - values: weights w in [-8, 7] as the fp6 e3m2 code of 2w (sign, 3 exponent bits of bias 3, 2 mantissa bits);
 *   activations q in [-8, 15] as the fp6 e2m3 code of q / 2 (bias 1, 3 mantissa bits). Both exact; the matrix
 *   cores multiply them at the fp6 rate and (2w)(q/2) = wq.
 * - bits: value k of a row's 64-deep group in half h = k / 32 at position i = k % 32; the 32 codes of a half packed
 *   little-endian, code i at bits [6i, 6i + 6) of 24 bytes.
 * - bytes: a row's group is 48 bytes [half 0 bytes 0..15][half 1 bytes 0..15][half 0 bytes 16..23][half 1 bytes
 *   16..23]; the matrix is [R/128][K/64][128][48], group g of row r at (r/128)*(K/64)*6144 + g*6144 + (r%128)*48,
 *   so the group of a 128-row tile that one GEMM step reads is one contiguous 6 KB block. */

/* Weight operand of the W4A4 GEMM: packed int4 weights qweight uint8 [N, K/2] (per 64-group, byte j holds k = j in
 * the low nibble and k = j + 32 in the high nibble, two's complement) -> the fp6 codes of the same integers in the
 * operand format (N * K * 3/4 bytes). N % 128 == 0. Done once per weight (module construction), the
 * expansion of the int4 weights that Nunchaku's gemm_w4a4 performs inside every call
 * (native/ops/w4a4_ops.cpp:36-38). 16-byte aligned buffers. */
int wdl_w4a4_weight_codes(const void* qweight, int64_t N, int64_t K, void* codes, wdl_stream_t stream);

/* Weight-scale operand of the W4A4 GEMM: n scales (bf16, or fp16 when fp16 != 0) -> n bf16 pairs packed in 32 bits,
 * hi | lo << 16, hi + lo = the scale exactly (hi the scale truncated to bf16, lo the rest: (s, 0) for a bf16 scale,
 * two exact bf16 parts for an fp16 one). The GEMM forms ws * as from both parts on the matrix cores, so fp16 weight
 * scales cost no extra work (the reference keeps bf16 scales, quantization/w4a4.py:171-174; fp16 is the other mode
 * Nunchaku's kernels accept). Done once per weight. scales 2-byte, pairs 4-byte aligned; finite scales. */
int wdl_w4a4_scale_pairs(const void* scales, int fp16, int64_t n, void* pairs, wdl_stream_t stream);

/* W4A4 GEMM with fused dequantization, low-rank up projection and bias. Replaces Nunchaku's gemm_w4a4 behind
 * live::w4a4_linear and live::w4a4_gelu_mlp (native/ops/w4a4_ops.cpp:36-38, 55-61).
 * y[m][n] = sum_g ascales[g][m] wscales[g][n] I_g[m][n] + bf16(lora[m]) . proj_up[n] + bias[n], I_g the exact
 * integer sum over the 64-group g. qa: [Mp, K] activation codes (wdl_act_quant_w4); wcodes: [N, K] weight codes
 * (wdl_w4a4_weight_codes), both in the operand format above; wscales [K/64, N] scale pairs (wdl_w4a4_scale_pairs);
 * lora fp32 [Mp, 32] or NULL; proj_up bf16 [N, 32]; bias bf16 [N] or NULL. epilogue: 0 out bf16 [M, ldo] = y;
 * 1 out fp32 = y; 2 out bf16 =
 * bf16(out + bf16(y) * gate[n]) in place (gated residual; gate fp32 [N]); 3 out bf16 = GELU_tanh(y).
 * Mp % 128 == 0, N % 128 == 0, K % 64 == 0, K <= 2^30; qa, wcodes, out, proj_up, lora, gate and workspace 16-byte
 * aligned, bias 8-byte, scales 4-byte; bf16 outputs: ldo % 8 == 0.
 * workspace: wdl_w4a4_gemm_workspace_bytes(Mp, N, K) bytes (no initial contents), or NULL. When the size is not 0
 * the product runs split in K over one workgroup per CU, for shapes whose tiles leave CUs idle: either the balanced
 * form (whole tiles dealt evenly, each summed by two halves of K, the few leftover tiles in 32 x 32 pieces summed
 * by eighths of K; one launch, the size is then a 256-byte token the kernel does not touch) or stream-K (the
 * (tile, group) iterations shared evenly, partial sums in the workspace added in a fixed order by a second
 * launch). Both are deterministic, their rounding not identical to the one-pass launch. With NULL the one-pass
 * launch runs. Calls sharing a workspace must not overlap.
 * ln_partials (epilogue 2 only, else NULL): fp32 [M][N / 32][2], 16-byte aligned, receives the LayerNorm chunk
 * partials of the rows written (the N columns being whole rows), in wdl_act_quant_w4's order, so the next
 * LayerNorm-fused quantization of out skips its statistics pass. No counterpart in the reference (its LayerNorm
 * is a separate torch op). */
int64_t wdl_w4a4_gemm_workspace_bytes(int64_t Mp, int64_t N, int64_t K);
int wdl_w4a4_gemm(const void* qa, const void* ascales, const void* wcodes, const void* wscales, const float* lora,
                  const void* proj_up, const void* bias, int64_t M, int64_t Mp, int64_t N, int64_t K, int64_t rank,
                  void* out, int64_t ldo, int epilogue, const float* gate, float* ln_partials, void* workspace,
                  wdl_stream_t stream);

/* Workspace (in floats) of wdl_w4a4_gemm_gelu_quant for Mp tokens and a hidden layer of N features. */
int64_t wdl_w4a4_gemm_gelu_quant_workspace_floats(int64_t Mp, int64_t N);

/* The first GEMM of the fused W4A4 GELU MLP with the second layer's input quantization in its epilogue. Replaces
 * the first gemm_w4a4 call of live::w4a4_gelu_mlp (native/ops/w4a4_ops.cpp:42-57; Nunchaku's fused_gelu_mlp as
 * quantization/w4a4.py:198-204 describes it: the hidden layer never goes to memory in 16 bits).
 * y as wdl_w4a4_gemm computes it (qa, ascales, wcodes, wscales, lora, proj_up, bias; N = the hidden width), then
 * per token m < M: h = GELU_tanh(y) in fp32; u = (h + 0.171875) / smooth2 (IEEE fp32 quotient); per 64-feature
 * group scale = bf16(max|u| / 15), q = clamp(rint(u / scale), 0, 15). Outputs, the inputs of the second layer's
 * wdl_w4a4_gemm: q2 the fp6 codes of q in the operand format [Mp, N], ascales2 bf16 [N/64, Mp], lora2 fp32
 * [Mp, 32] = h . proj_down2 (rows >= M: zero codes, scales and sums). smooth2 bf16 [N]; proj_down2_t bf16 [32, N].
 * The low-rank sum is formed per 128-feature tile (h split exactly into two bf16 parts for the matrix cores) and
 * the tiles are added in increasing order by a second launch: deterministic. workspace: fp32,
 * wdl_w4a4_gemm_gelu_quant_workspace_floats(Mp, N). Mp % 128 == 0, N % 128 == 0, K % 64 == 0; codes, lora,
 * lora2, proj_up and workspace 16-byte aligned, bias, smooth2 and proj_down2_t 8-byte, scales 4-byte. */
int wdl_w4a4_gemm_gelu_quant(const void* qa, const void* ascales, const void* wcodes, const void* wscales,
                             const float* lora, const void* proj_up, const void* bias, int64_t M, int64_t Mp,
                             int64_t N, int64_t K, int64_t rank, const void* smooth2, const void* proj_down2_t,
                             void* q2, void* ascales2, float* lora2, float* workspace, wdl_stream_t stream);

/* Workspace (in floats) of wdl_fp8_quantize in per-tensor mode for an [M, K] operand. */
int64_t wdl_fp8_quantize_workspace_floats(int64_t M, int64_t K);

/* FP8 E4M3 quantization of a linear-layer operand. Replaces quantize and quantize_rows
 * (src/wan_dit_lab/quantization/fp8.py:14-17, 37-41) as Fp8Linear, DynamicFp8Linear and PackedFp8Linear use them
 * (fp8.py:20-94). x: bf16 (x_dtype 2) or fp32 (0) [M, K], row stride ldx (16-byte aligned rows), K % 16 == 0.
 * rows != 0: scale[m] = max(max_k |x[m][k]|, 1e-12) / 448 (scale fp32 [Mp]); rows == 0: one scale for the tensor
 * (scale fp32 [1], workspace: wdl_fp8_quantize_workspace_floats(M, K)). q [Mp, K] = e4m3(x / scale) (IEEE quotient,
 * round to nearest even), rows M..Mp-1 zero (scale 0). Deterministic (no atomics). */
int wdl_fp8_quantize(const void* x, int x_dtype, int64_t ldx, int64_t M, int64_t K, int64_t Mp, int rows, void* q,
                     float* scale, float* workspace, wdl_stream_t stream);

/* FP8 GEMM with torch._scaled_mm's scaled epilogue. Replaces the _scaled_mm calls of Fp8Linear,
 * DynamicFp8Linear and PackedFp8Linear (src/wan_dit_lab/quantization/fp8.py:32-33, 60-66, 92-93; cuBLASLt there).
 * xq: e4m3 [Mp, K] (wdl_fp8_quantize), wq: e4m3 [N, K] ([out, in]); acc = sum_k xq[m][k] wq[n][k] in fp32.
 * rows != 0: out = bf16(float(bf16(acc)) * (x_scale[m] * w_scale[n]) + bias[n]) (fp8.py:57-62);
 * rows == 0: out = bf16(acc * (x_scale[0] * w_scale[0]) + bias[n]) (one rounding). bias bf16 [N] or NULL;
 * out bf16 [M, ldo]. Mp % 128 == 0, N % 128 == 0, K % 64 == 0, operands 16-byte aligned.
 * workspace: wdl_fp8_gemm_workspace_bytes(Mp, N, K) bytes (16-byte aligned, no initial contents), or NULL. When
 * the size is not 0 and a workspace is given, the product is split in K over one workgroup per CU (stream-K:
 * fp32 partial sums of each tile's pieces added in a fixed order), which changes the fp32 summation order of the
 * one-pass launch: deterministic, not bit-identical to it. */
int64_t wdl_fp8_gemm_workspace_bytes(int64_t Mp, int64_t N, int64_t K);
int wdl_fp8_gemm(const void* xq, const float* x_scale, const void* wq, const float* w_scale, const void* bias,
                 int64_t M, int64_t Mp, int64_t N, int64_t K, int rows, void* out, int64_t ldo, void* workspace,
                 wdl_stream_t stream);

/* FP8 weight-only linear: out = bf16(w_scale[n] * sum_k x[m][k] w[n][k] + bias[n]) (epilogue 0), or the gated
 * residual out = bf16(out + bf16(y) * gate[n]) in place (epilogue 2). x bf16 [M, ldx] (ldx % 8 == 0), w e4m3 [N, K]
 * row-major, w_scale fp32 [N] (scale_rows != 0) or [1], bias bf16 [N] or NULL, gate fp32 [N]; out bf16 [M, ldo]
 * (ldo % 4 == 0). Products of bf16 and e4m3 values are exact; sums in fp32 on the bf16 matrix cores. N % 128 == 0,
 * K % 64 == 0; x and w 16-byte aligned, out 8-byte. No counterpart in the reference, whose FP8 linears are W8A8
 * (quantization/fp8.py:1-6): the attention projections of the benchmark's mixed-precision mode. */
int wdl_fp8wo_gemm(const void* x, int64_t ldx, const void* w, const float* w_scale, int scale_rows, const void* bias,
                   int64_t M, int64_t N, int64_t K, void* out, int64_t ldo, int epilogue, const float* gate,
                   wdl_stream_t stream);

/* Q/K RMSNorm over all heads + 3D RoPE, fused. Replaces norm_q / norm_k (src/wan_dit_lab/models/rms_norm.py:10-13,
 * used at src/wan_dit_lab/quantization/w4a4.py:256-257) and rope_apply / wan_dit_lab::rope3d_rotate
 * (src/wan_dit_lab/models/rope.py:12-31; src/wan_dit_lab/kernels/rope_triton.py:66-81, 101-144).
 * q, k: bf16 [M, heads*128] with row strides ldq, ldk; wq, wk: bf16 [heads*128] or NULL (then that input is only
 * rotated: rope_apply alone); k may be NULL (q only). freq: [2, positions, 64] (cos, sin; pairs split [22 time,
 * 21 height, 21 width]) of type freq_dtype (0 fp32, 3 fp64); grid (f, h, w) with f*h*w <= M, time offset
 * start_frame. Row m: n = bf16(x * rstd), y = bf16(n * w); pairs of rows m < f*h*w rotated at (start_frame +
 * m/(h*w), (m/w)%h, m%w) in the table's precision (fp64 results rounded to fp32, then bf16), results bf16 into
 * q_out, k_out [M, heads*128] (row stride ldo). */
int wdl_qk_norm_rope(const void* q, int64_t ldq, const void* k, int64_t ldk, const void* wq, const void* wk,
                     const void* freq, int freq_dtype, int64_t positions, int64_t M, int64_t heads, int f, int h,
                     int w, int start_frame, float eps, void* q_out, void* k_out, int64_t ldo, wdl_stream_t stream);

/* The standalone 3D RoPE rotation. Replaces wan_dit_lab::rope3d_rotate (src/wan_dit_lab/kernels/rope_triton.py:14-81)
 * and rope_apply (rope_triton.py:84-139; models/rope.py:12-31). x: [B, L, H, dim] of type x_dtype (0 fp32, 1 fp16,
 * 2 bf16, 3 fp64) with element strides x_strides[4]; freq: [2, positions, dim/2] (cos, sin) fp32 or fp64 with
 * element strides freq_strides[3]; grids: host int32 [B][3] (f, h, w) per sample, 1 <= B <= 64; even dim.
 * Pair p of token i of sample b (i < f h w) turns by the table's angle at: start + i / (h w) for the first
 * dim/2 - 2 ((dim/2) / 3) pairs (time), (i / w) % h for the next (dim/2) / 3 (height), i % w for the rest
 * (width); (e, o) -> (e c - o s, o c + e s), s negated when inverse != 0. Arithmetic in fp64 if x or freq is fp64,
 * else fp32, each product rounded; fp16 / bf16 results through fp32. Tokens i >= f h w are copied. out: contiguous
 * [B, L, H, dim] of out_dtype. Grids that exceed L or the table are rejected before the launch. */
int wdl_rope3d_rotate(const void* x, int x_dtype, const int64_t* x_strides, const void* freq, int freq_dtype,
                      const int64_t* freq_strides, int64_t positions, int64_t B, int64_t L, int64_t H, int64_t dim,
                      const int32_t* grids, int64_t start, int inverse, void* out, int out_dtype,
                      wdl_stream_t stream);

/* Sage per-thread int8 quantization of Q. Replaces sage_kv.quant_q (src/wan_dit_lab/kernels/sage_kv.py:112-124).
 * x: bf16 [n, heads, 128] (token stride ldx); q: int8 [n, heads, 128]; q_scale: fp32 [heads, ceil(n/128)*32].
 * Per 32-token block, tokens l, l+8, l+16, l+24 share scale = max|x| / 127 + 1e-7; q = trunc(x/scale +- 0.5). */
int wdl_quant_q(const void* x, int64_t ldx, int64_t n, int64_t heads, void* q, float* q_scale, wdl_stream_t stream);

/* Workspace (in floats) that wdl_sage_prep needs for `splits` token splits. */
int64_t wdl_sage_prep_workspace_floats(int64_t heads, int splits);

/* Sage preparation straight from the FP8 cache: K mean, int8 K, fp8 V. Replaces the Triton kernels _sum_max,
 * _quant_k, _quant_v of sage_kv._attend (src/wan_dit_lab/kernels/sage_kv.py:43-105, 152-173).
 * Tokens t < at from cache_k/cache_v (fp8 [capacity, heads, 128]) times cache_ks/cache_vs (fp32 [capacity, heads]),
 * at <= t < at + n from k, v (bf16 [n, heads, 128], token strides ldk, ldv). Outputs: k_int8 [heads, Lpad, 128],
 * k_scale fp32 [heads, Lpad/16], v_fp8 [heads, 128, Lpad] (within each 64-token block, token t at position
 * 32*((t%8)/4) + 4*(t/8) + t%4), Lpad = 64*ceil(L/64); k_mean_out / v_scale_out fp32 [heads, 128] (may be NULL:
 * then kept in the workspace). Batch 1. */
int wdl_sage_prep(const void* cache_k, const float* cache_ks, const void* cache_v, const float* cache_vs,
                  int64_t capacity, const void* k, int64_t ldk, const void* v, int64_t ldv, int64_t heads, int64_t at,
                  int64_t n, int splits, float* workspace, void* k_int8, float* k_scale, void* v_fp8,
                  float* k_mean_out, float* v_scale_out, wdl_stream_t stream);

/* wdl_sage_prep with the head and token maps of sage_kv.attend (src/wan_dit_lab/kernels/sage_kv.py:127-134, 137-140;
 * used by KVCache.attend_split, generation/causal.py:222-241): the cache holds cache_heads >= heads heads; head h of
 * the call reads cache head heads_map[h] (int32 [heads], device; NULL: h, and then cache_heads == heads); cached
 * token t < at is cache row tokens_map[t] (int32 [at], device; NULL: t). Neither copies the cache. Map values outside
 * [0, cache_heads) / [0, capacity) are clamped into the cache by the kernels (the host wrapper rejects them first). */
int wdl_sage_prep_mapped(const void* cache_k, const float* cache_ks, const void* cache_v, const float* cache_vs,
                         int64_t capacity, int64_t cache_heads, const int32_t* heads_map, const int32_t* tokens_map,
                         const void* k, int64_t ldk, const void* v, int64_t ldv, int64_t heads, int64_t at,
                         int64_t n, int splits, float* workspace, void* k_int8, float* k_scale, void* v_fp8,
                         float* k_mean_out, float* v_scale_out, wdl_stream_t stream);

/* Statistics of the cached tokens [0, at) for wdl_sage_prep_cached: stats fp32 [2, heads, 128] = the K column sums
 * (`splits` token splits, each summed in a fixed order, then added in split order) and the |V| column maxima, of
 * cache rows 0 .. at-1 (e4m3 value times the row's scale). No counterpart in the reference, whose _sum_max pass
 * (src/wan_dit_lab/kernels/sage_kv.py:43-60) re-reads every cached token at every call: the statistics change only
 * when the cache's rows [0, at) do, so KVCache refreshes them at a commit. workspace: wdl_sage_prep_workspace_floats
 * floats. Batch 1; at = 0 gives zeros. */
int wdl_sage_cache_stats(const void* cache_k, const float* cache_ks, const void* cache_v, const float* cache_vs,
                         int64_t capacity, int64_t heads, int64_t at, int splits, float* workspace, float* stats,
                         wdl_stream_t stream);

/* wdl_sage_prep with the cached tokens' statistics from wdl_sage_cache_stats (same cache, same at): the statistics
 * pass reads only the chunk's n tokens, k_mean = (cached K sums + the chunk's, in split order) / (at + n),
 * v_scale = max(cached |V| maxima, the chunk's, 1e-8) / 2.25; the quantization is wdl_sage_prep's. The K mean
 * differs from wdl_sage_prep's only in the fp32 summation order. */
int wdl_sage_prep_cached(const void* cache_k, const float* cache_ks, const void* cache_v, const float* cache_vs,
                         int64_t capacity, const void* k, int64_t ldk, const void* v, int64_t ldv, int64_t heads,
                         int64_t at, int64_t n, const float* cache_stats, int splits, float* workspace, void* k_int8,
                         float* k_scale, void* v_fp8, float* k_mean_out, float* v_scale_out, wdl_stream_t stream);

/* wdl_sage_prep_cached that also appends the chunk to the caches: rows at .. at + n - 1 of cache_k / cache_v (fp8
 * [capacity, heads, 128]) and cache_ks / cache_vs (fp32 [capacity, heads]) receive k, v as wdl_kv_append_fp8 writes
 * them (the same bytes and scales), from the values the quantization pass already holds, so the chunk is read once
 * and the append needs no launch of its own. Replaces KVCache.store followed by KVCache.attend's preparation
 * (src/wan_dit_lab/generation/causal.py:177-181, 193-220; kernels/cache_fp8.py:59-72 and sage_kv.py:127-134).
 * Requires at + n <= capacity; rows [0, at) are only read, rows [at, at + n) only written. */
int wdl_sage_prep_cached_append(void* cache_k, float* cache_ks, void* cache_v, float* cache_vs, int64_t capacity,
                                const void* k, int64_t ldk, const void* v, int64_t ldv, int64_t heads, int64_t at,
                                int64_t n, const float* cache_stats, int splits, float* workspace, void* k_int8,
                                float* k_scale, void* v_fp8, float* k_mean_out, float* v_scale_out,
                                wdl_stream_t stream);

/* The operands live::sage_sm89 receives from the reference's sage_kv._attend (kernels/sage_kv.py:141-176; schema
 * native/ops/sage_ops.cpp:12-19, 28-31) in wdl_sage_attn's layouts: k_i8 int8 [L, heads, 128] (row stride ldk
 * bytes) -> k_out int8 [heads, Lpad, 128], tokens L..Lpad-1 zero; v_fp8 e4m3 [128, heads, Lpad] (element strides
 * v_stride_d, v_stride_h, tokens contiguous) in Sage's 16-token order (sage_kv.py:101-103) -> v_out [heads, 128,
 * Lpad] in wdl's 64-token order. Lpad = 64 ceil(L / 64). q_scale, k_scale and v_scale already have wdl's layouts.
 * Pointers and strides 16-byte aligned. */
int wdl_sage_sm89_relayout(const void* k_i8, int64_t ldk, const void* v_fp8, int64_t v_stride_d, int64_t v_stride_h,
                           int64_t L, int64_t heads, void* k_out, void* v_out, wdl_stream_t stream);

/* Workspace (bytes) of wdl_sage_attn for n queries, L keys and `heads` heads. */
int64_t wdl_sage_attn_workspace_bytes(int64_t n, int64_t L, int64_t heads);

/* Sage-2 style attention (int8 QK^T, fp32 online softmax, fp8 PV, non-causal). Replaces live::sage_sm89
 * (native/ops/sage_ops.cpp:12-19, 28-35) on the layouts of wdl_quant_q / wdl_sage_prep.
 * out: bf16 [n, heads, 128] (row stride ldo). workspace: 16-byte aligned, wdl_sage_attn_workspace_bytes(n, L,
 * heads) bytes (no initial contents needed); calls that share a workspace must not overlap. When the (128-query
 * tile, head) pairs just exceed a multiple of the CU count, every CU runs the same number of whole tiles and the
 * key blocks of the remaining tiles are split evenly over half the CUs; their partial softmax states go through the
 * workspace to a second launch that merges them in a fixed order (deterministic). Otherwise the workspace is not
 * touched and may be NULL. */
int wdl_sage_attn(const void* q_i8, int64_t ldq, const float* q_scale, const void* k_i8, const float* k_scale,
                  const void* v_fp8, const float* v_scale, int64_t n, int64_t L, int64_t heads, float sm_scale,
                  void* out, int64_t ldo, void* workspace, wdl_stream_t stream);

/* wdl_sage_attn with Q given in bf16 [n, heads, 128] (row stride ldq): the kernel quantizes it by Sage's per-thread
 * int8 rule of wdl_quant_q (kernels/sage_kv.py:112-124) as it loads each query tile, so the result is bit-identical
 * to wdl_quant_q followed by wdl_sage_attn, without the int8 Q round trip through memory. Replaces the pair
 * quant_q + live::sage_sm89 that sage_kv_attend runs (kernels/sage_kv.py:170-176). Same workspace rules. */
int wdl_sage_attn_q16(const void* q_bf16, int64_t ldq, const void* k_i8, const float* k_scale, const void* v_fp8,
                      const float* v_scale, int64_t n, int64_t L, int64_t heads, float sm_scale, void* out,
                      int64_t ldo, void* workspace, wdl_stream_t stream);

/* wdl_sage_attn_q16 with a block-causal mask per latent frame: the n queries are the chunk, the last n of the L
 * keys (after L - n cached ones), and chunk query q sees keys [0, L - n + (q / frame_tokens + 1) frame_tokens), the
 * cache and the chunk's frames up to its own. No counterpart in the reference, whose chunk attention sees the whole
 * chunk (native/ops/sage_ops.cpp:15-16; generation/causal.py:269): the benchmark's chunk-causal attention mode.
 * frame_tokens > 0, n <= L; the workspace is not used (may be NULL): every (query tile, head) runs whole. */
int wdl_sage_attn_q16_framed(const void* q_bf16, int64_t ldq, const void* k_i8, const float* k_scale,
                             const void* v_fp8, const float* v_scale, int64_t n, int64_t L, int64_t heads,
                             float sm_scale, int64_t frame_tokens, void* out, int64_t ldo, void* workspace,
                             wdl_stream_t stream);

/* Elements (bf16) of each of the two operands wdl_attn_bf16_prep writes for L keys and `heads` heads. */
int64_t wdl_attn_bf16_prep_elems(int64_t L, int64_t heads);

/* The keys and values of a bf16 attention laid out for wdl_attn_bf16, once per prompt: K, V bf16 [L, heads, 128]
 * (token strides ldk, ldv; K rows 16-byte aligned) -> Kp bf16 [heads][Lpad][128] (each key row's 16-byte chunks
 * XOR-swizzled by key % 16) and Vp bf16 [heads][128][Lpad] (V transposed; in each 16-key group the keys ordered
 * 0..3, 8..11, 4..7, 12..15; each channel row's 16-byte chunks of a 64-key block XOR-swizzled by (channel / 2) % 8),
 * Lpad = 64 ceil(L / 64), keys >= L zero. Part of the cross-attention that keys_values and Stream.cross compute once
 * per prompt (models/multi_head_attention.py:21-26; generation/causal.py:557-568). */
int wdl_attn_bf16_prep(const void* k, int64_t ldk, const void* v, int64_t ldv, int64_t L, int64_t heads, void* kp,
                       void* vp, wdl_stream_t stream);

/* bf16 attention (non-causal, fp32 online softmax, P rounded to bf16 for the P V product, fp32 accumulation):
 * out = softmax(Q K^T sm_scale) V. Replaces torch.nn.functional.scaled_dot_product_attention on bf16 operands, as
 * the reference's cross-attention runs it (models/multi_head_attention.py:37-44 with the context's keys and values;
 * generation/causal.py:418-420). q: bf16 [n, heads, 128] (row stride ldq); kp, vp: wdl_attn_bf16_prep's layouts of
 * L keys; out bf16 [n, heads, 128] (row stride ldo). No workspace. */
int wdl_attn_bf16(const void* q, int64_t ldq, const void* kp, const void* vp, int64_t n, int64_t L, int64_t heads,
                  float sm_scale, void* out, int64_t ldo, wdl_stream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* WDL_H */
