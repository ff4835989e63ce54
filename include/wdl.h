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

#ifdef __cplusplus
}
#endif

#endif /* WDL_H */
