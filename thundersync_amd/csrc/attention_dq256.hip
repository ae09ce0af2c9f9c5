// Attention backward: dQ at head dim 256 (query-stationary, K/V tiles shared
// by the waves).  Four waves of 16 rows, one per SIMD, covering the work
// item's rows in two passes over its keys (the Q/dO rows and dQ accumulators
// of 32 rows per wave, or of 16 rows at two waves per SIMD, do not fit the
// registers); compiled with the default code generation (attention_dq.hip
// compiles the head-dim-128 instance with MFMA results in VGPRs).
#include "attention_dq_wave.h"

namespace ts {
namespace attn {

template <typename E>
void launch_dq_wave256_t(const ts_attn_problem& P, int gc, dim3 grid, ts_attn_rows q, ts_attn_rows dout,
                         const float* rowstats, int64_t lse_ld, ts_attn_rows dq, hipStream_t s) {
  ts::TimedLaunch timed_("attention.dq_kernel", s);
  if (gc == 4)
    hipLaunchKernelGGL((dq_wave_kernel<E, 1, 256, 4, 2>), grid, dim3(256), 0, s, P, q, dout, rowstats, lse_ld, dq);
  else if (gc == 2)
    hipLaunchKernelGGL((dq_wave_kernel<E, 1, 256, 2, 2>), grid, dim3(256), 0, s, P, q, dout, rowstats, lse_ld, dq);
  else
    hipLaunchKernelGGL((dq_wave_kernel<E, 1, 256, 1, 2>), grid, dim3(256), 0, s, P, q, dout, rowstats, lse_ld, dq);
}

void launch_dq_wave256(const ts_attn_problem& P, int gc, dim3 grid, ts_attn_rows q, ts_attn_rows dout,
                       const float* rowstats, int64_t lse_ld, ts_attn_rows dq, hipStream_t s) {
  if (P.dtype == kF16)
    launch_dq_wave256_t<f16>(P, gc, grid, q, dout, rowstats, lse_ld, dq, s);
  else
    launch_dq_wave256_t<bf16>(P, gc, grid, q, dout, rowstats, lse_ld, dq, s);
}

}  // namespace attn
}  // namespace ts
