/*
 * mi_model.h -- C ABI of the dense decoder-layer ops the engine runs around
 * the paged-KV attention path (libmi_attn.so, gfx950).
 *
 * These have no counterpart in the reference's FFI: the reference runs the
 * same math as torch in Python -- FuseLayerNorm (microinfer/layer/norm.py:
 * 20-35, fused by torch.compile in _compiled_add_rms_norm, norm.py:13-16),
 * the FFN's SwiGLU gate (_compiled_swiglu, microinfer/layer/transformer.py:
 * 12-15, called from FFN.forward :82-88) and every dense projection as
 * F.linear. The engine calls these instead at decode batch sizes, where a
 * step is made of many small launches and the projections are bound by
 * streaming their weights.
 *
 * Conventions are those of mi_attn.h: MI_OK or a non-zero status with
 * mi_last_error(); element strides; dtype MI_DTYPE_BF16 or MI_DTYPE_F16
 * (MI_ERR_UNSUPPORTED otherwise, so the caller can keep its torch path);
 * `stream` is a hipStream_t (NULL: the default stream). Every entry point is
 * one launch with no allocation and no memset, so it can be captured into a
 * hipGraph.
 */
#ifndef MI_MODEL_H_
#define MI_MODEL_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/*
 * y[m, n] = sum_k x[m, k] * w[n, k] (torch's F.linear without bias), float32
 * accumulation, one rounding to the element type. For m <= 64 (decode
 * batches): each weight row streams through MFMA once; a workgroup's waves
 * split k and add their sums in a fixed order (deterministic).
 * n % 16 == 0, k % 32 == 0, every pointer and row stride 16-byte aligned.
 * m > 64 returns MI_ERR_UNSUPPORTED.
 */
int32_t mi_linear(const void* x, int64_t x_row_stride, const void* w, int64_t w_row_stride,
                  void* y, int64_t y_row_stride, int32_t m, int32_t n, int32_t k,
                  int32_t dtype, void* stream);

/*
 * The FFN's gate/up projection with its SwiGLU gate (FFN.forward,
 * microinfer/layer/transformer.py:82-88: gate_up = F.linear(x, w), then
 * _compiled_swiglu :12-15): w holds 2 * inter rows, the gate's then the up
 * projection's; y[m, inter] = round(round(silu(g)) * u) with
 * g = round(x . w[c]^T), u = round(x . w[inter + c]^T) -- mi_linear followed
 * by mi_silu_mul, bit for bit, in one launch that writes only y.
 * inter % 16 == 0, k % 32 == 0, every pointer and row stride 16-byte
 * aligned; m > 64 returns MI_ERR_UNSUPPORTED.
 */
int32_t mi_linear_swiglu(const void* x, int64_t x_row_stride, const void* w,
                         int64_t w_row_stride, void* y, int64_t y_row_stride, int32_t m,
                         int32_t inter, int32_t k, int32_t dtype, void* stream);

/*
 * FuseLayerNorm's forward (microinfer/layer/norm.py:26-35) on `rows` rows:
 * s = x + residual (rounded to the element type; s = x when residual is
 * NULL), residual_out = s (skipped when residual_out is NULL), and
 * out = round(round(s * rsqrt(mean(s^2) + eps)) * weight) -- the rounding
 * steps of torch's rms_norm on 16-bit inputs. dim % 8 == 0, dim <= 8192,
 * pointers and strides 16-byte aligned. out may alias x; residual_out may
 * alias x or residual.
 */
int32_t mi_rms_norm_residual(const void* x, int64_t x_row_stride, const void* residual,
                             int64_t residual_row_stride, const void* weight, float eps,
                             void* out, int64_t out_row_stride, void* residual_out,
                             int64_t residual_out_row_stride, int32_t rows, int32_t dim,
                             int32_t dtype, void* stream);

/*
 * SwiGLU gate: out[r, i] = round(round(silu(gate[r, i])) * up[r, i]) with
 * gate = gate_up[r, 0:inter] and up = gate_up[r, inter:2 inter] (the rounding
 * steps of torch's F.silu(gate) * up on 16-bit tensors). inter % 8 == 0,
 * pointers and strides 16-byte aligned.
 */
int32_t mi_silu_mul(const void* gate_up, int64_t gate_up_row_stride, void* out,
                    int64_t out_row_stride, int32_t rows, int32_t inter, int32_t dtype,
                    void* stream);

#ifdef __cplusplus
} /* extern "C" */
#endif

#endif /* MI_MODEL_H_ */
