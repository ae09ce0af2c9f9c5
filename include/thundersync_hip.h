/*
 * thundersync_hip.h -- C ABI of libthundersync_hip.so, the MI355X (gfx950)
 * kernels behind thundersync_amd's operators.
 *
 * Conventions (all entry points):
 *   - every tensor argument is a raw device pointer; sizes and strides are
 *     int64 element counts; `stream` is a hipStream_t passed as void*;
 *   - the caller (PyTorch on the host side) allocates every input, output
 *     and workspace; the library never allocates, frees or retains memory;
 *   - inputs are never written, so a call may be repeated on the same
 *     inputs (activation-checkpoint recompute does exactly that);
 *   - the return value is a status (TS_OK or a TS_ERR_* code); the message
 *     of the last failure on the calling thread is ts_hip_last_error().
 *
 * Each declaration names the reference interface it replaces.  Paths are
 * relative to the reference repository root (seilk/thundersync,
 * src/thundersync/...).
 */
#ifndef THUNDERSYNC_HIP_H
#define THUNDERSYNC_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define TS_OK 0
#define TS_ERR_INVALID 1   /* bad argument: shape, dtype, alignment, size */
#define TS_ERR_LAUNCH 2    /* the HIP runtime refused a launch */
#define TS_ERR_DEVICE 3    /* the current device is not a gfx950 */

/* dtype codes */
#define TS_F32 0
#define TS_F16 1
#define TS_BF16 2

/* Library version string, e.g. "thundersync_hip 0.1.0 gfx950". */
const char* ts_hip_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* ts_hip_last_error(void);

/* ------------------------------------------------------------------------
 * RMSNorm
 * ------------------------------------------------------------------------ */

/* Forward with the replaced Qwen3RMSNorm's operation order and casts:
 *   xf = float(x); rstd = rsqrt(mean(xf^2) + eps);
 *   y = w * T(xf * rstd)            (product rounded to T, as torch does)
 * x, y: [rows, width] of dtype; w: [width] of dtype; rstd: [rows] fp32.
 * Replaces FP32RMSNormVJP.forward (accel/rms_norm.py:9-17) and the compiled
 * primal `_primal` / `_CompiledForwardVJP` (grpo/rms_norm.py:12-31). */
int ts_rmsnorm_fwd(const void* x, const void* w, void* y, float* rstd,
                   int64_t rows, int64_t width, float eps, int dtype,
                   void* stream);

/* Workspace bytes ts_rmsnorm_bwd needs for `rows` x `width`. */
int64_t ts_rmsnorm_bwd_workspace(int64_t rows, int64_t width);

/* FP32 VJP from the saved statistic:
 *   xhat = float(x) * rstd;  g = float(dy) * float(w)
 *   dx = T(rstd * (g - xhat * mean(g * xhat)))
 *   dw = T(sum_rows float(dy) * float(x) * rstd)
 * dx or dw may be NULL when that gradient is not needed.  The dw sum is a
 * fixed-order reduction: identical inputs give identical bits.
 * Replaces FP32RMSNormVJP.backward (accel/rms_norm.py:19-43, the
 * aten._fused_rms_norm_backward call at :28) and
 * native_source_rms_backward with its Triton dW kernels
 * (grpo/rms_norm_native.py:8-74). */
int ts_rmsnorm_bwd(const void* dy, const void* x, const void* w,
                   const float* rstd, void* dx, void* dw, void* workspace,
                   int64_t workspace_bytes, int64_t rows, int64_t width,
                   int dtype, void* stream);

/* ------------------------------------------------------------------------
 * Diagnostics
 * ------------------------------------------------------------------------ */

/* Runs one v_mfma_f32_16x16x32_bf16 and one v_mfma_f32_32x32x16_bf16 on
 * operands the caller lays out per lane (a, b: 64 lanes x 8 bf16 each), and
 * the 8x8 16-bit register transpose on `t_in` (64 lanes x 8 x 8 bf16).
 * Writes d16: 64 x 4 fp32, d32: 64 x 16 fp32, t_out: 64 x 8 x 8 bf16.
 * Used by the test suite to pin the lane layouts the kernels assume. */
int ts_probe_layouts(const void* a, const void* b, float* d16, float* d32,
                     const void* t_in, void* t_out, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* THUNDERSYNC_HIP_H */
