/*
 * dan_fp8.h -- C ABI of the gfx950 e4m3 quantizer for dan's FP8 decoder
 * linears.
 *
 * dan's FP8Linear (dan/quant.py:23-42) quantizes its weight once (per output
 * row, or per tensor) and its input on every call with fp8_quantize
 * (dan/fused.py:85-91):
 *     amax  = max |x|  over each row (rowwise) or over the whole tensor
 *     scale = max(amax, 1e-12) / 448            (fp32)
 *     xq    = e4m3fn(x / scale)                  (fp32 divide, round to nearest even)
 * and then multiplies with torch._scaled_mm (dan/quant.py:40), a library fp8
 * GEMM with the two scale vectors and the bias in its epilogue. On gfx950 that
 * GEMM is hipBLASLt's (OCP e4m3, v_mfma_*_f8f6f4); this library supplies the
 * quantizer: one read of x and one write of xq per call (rowwise), where the
 * eager chain makes five passes.
 *
 * Conventions are those of dan_tree_attn.h: caller-owned device memory,
 * nothing allocated or kept, asynchronous on `stream`, 0 on success and a
 * DanStatus with dan_tree_attn_last_error() on failure.
 */
#ifndef DAN_FP8_H
#define DAN_FP8_H

#include <stdint.h>

#include "dan_tree_attn.h"

#ifdef __cplusplus
extern "C" {
#endif

#define DAN_FP8_ABI_VERSION 1

typedef enum {
  DAN_FP8_SCALE_TENSOR = 0, /* one scale for the whole tensor (dan's sm89 mode) */
  DAN_FP8_SCALE_ROW = 1     /* one scale per row (dan's default on sm90+) */
} DanFp8ScaleMode;

typedef struct {
  int32_t abi_version; /* DAN_FP8_ABI_VERSION */
  int32_t dtype;       /* DanDtype of x: bf16, f16 or f32 */
  int32_t rows;        /* M */
  int32_t cols;        /* K: a multiple of 16 */
  int32_t mode;        /* DanFp8ScaleMode */
  int32_t reserved;
  const void *x;       /* [M, K], row stride x_stride elements, 16-byte aligned rows */
  int64_t x_stride;
  uint8_t *xq;         /* [M, K] e4m3fn (OCP) codes, row-major, row stride K */
  float *scale;        /* [M] (rowwise) or [1] (tensor) fp32 */
} DanFp8QuantArgs;

/* Quantize x to e4m3fn with dan's scale convention.
 * Replaces dan/fused.py:85-91 (fp8_quantize) on gfx950. */
int dan_fp8_quantize(const DanFp8QuantArgs *args, void *stream);

int dan_fp8_abi_version(void);

#ifdef __cplusplus
}
#endif

#endif /* DAN_FP8_H */
