/* Fused per-layer steps of the end-to-end decode harness (reskv_amd/llama.py).
 *
 * These are not ResKV operators and have no counterpart in the reference's
 * kernels: the reference's model patch runs them as chains of torch ops
 * (reskv/models/llama.py:37-43 and the transformers Llama layer it wraps:
 * RMSNorm, rotary embedding, gated MLP).  The harness uses them so that a
 * decode step of a batch-16 Llama-3.1-8B-shaped model is not dominated by
 * dozens of tiny elementwise launches per layer; every one of them is
 * compared with the torch formula it replaces in tests/test_gpu_llama_ops.py.
 *
 * Conventions as in reskv_hip.h: fp16 tensors are passed as void*, every
 * call returns 0 on success and non-zero on error (reskv_last_error() says
 * why), and `stream` is a hipStream_t (NULL: the null stream). */
#ifndef RESKV_LLAMA_H
#define RESKV_LLAMA_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* y[r] = fp16(fp32(x[r]) * rsqrt(mean(fp32(x[r])^2) + eps) * fp32(w)) for rows
 * r < rows of `hidden` fp16 values (hidden a multiple of 8, at most 8192;
 * x, w and y 16-byte aligned and contiguous). */
int reskv_llama_rmsnorm(const void* x, const void* w, void* y, int rows, int hidden, float eps, void* stream);

/* out[r, j] = fp16(fp32(fp16(silu(fp32(gu[r, j])))) * fp32(gu[r, ffn + j])):
 * gu fp16 [rows, 2*ffn] (gate then up), out fp16 [rows, ffn]; ffn a multiple
 * of 8, both contiguous and 16-byte aligned. */
int reskv_llama_silu_mul(const void* gu, void* out, int rows, int ffn, void* stream);

/* Splits the fused QKV projection of one token per batch row, rotates Q and K
 * and appends K/V to a cache:
 *   qkv fp16 [B, (Hq + 2 Hk) * 128] (Q heads, then K, then V);
 *   cos/sin fp32 [*, 64], row *pos (device int64) used for the rotation
 *   r = fp16(cat(a*c - b*s, b*c + a*s)) of halves a, b of a head, each product
 *   and sum rounded to fp32 (no fused multiply-add);
 *   q, qr fp16 [B, Hq, 128] (raw and rotated), k, kr, v fp16 [B, Hk, 128];
 *   append (each may be NULL): cache_rot <- kr, cache_raw <- k, cache_v <- v
 *   at token *slot (device int64) of fp16 [B, Hk, cap, 128] tensors with the
 *   given element strides for batch, head and token (channel stride 1). */
int reskv_llama_qkv_rope(const void* qkv, const float* cos, const float* sin, const int64_t* pos, int B,
                         int Hq, int Hk, void* q, void* qr, void* k, void* kr, void* v, void* cache_rot,
                         void* cache_raw, void* cache_v, const int64_t* slot, int64_t stride_b,
                         int64_t stride_h, int64_t stride_t, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* RESKV_LLAMA_H */
