// The split-K MFMA linear layer of the prefill (prefill.hip) as host launchers, shared with the
// multi-stream decode (streams.hip). Y = X W^T: X f32 [M][ldx], W f16 [N][K] (nn.Linear layout);
// partial sums over S K-splits go to part [S][M][ldp] at columns p_off..p_off+N and are summed in
// split order by one of the finish launchers, which also apply the epilogue.
#pragma once

#include <hip/hip_runtime.h>

#include <cstddef>
#include <cstdint>

namespace navi_amd {
namespace pf {

int pick_splits(int M, int K, int N);
size_t splits_floats(int M, int K, int N);
void launch_partial(const float *x, int ldx, int M, const uint16_t *w, int K, int N, int S, float *part, int ldp, int p_off,
                    uint32_t *flag, hipStream_t st);
// The same over W given as up to three row blocks w0 [n0][K] | w1 [n1][K] | w2 [n2][K] (each a
// multiple of 64 rows; n1 = n2 = 0 for one block), e.g. q | k | v in one launch.
void launch_partial3(const float *x, int ldx, int M, const uint16_t *w0, int n0, const uint16_t *w1, int n1, const uint16_t *w2,
                     int n2, int K, int S, float *part, int ldp, int p_off, uint32_t *flag, hipStream_t st);
// x[m] = (S > 0 ? sum_s part + x[m] : src[m]); xn[m] = RMSNorm(x[m]) * w; H == 1024.
void launch_resid_norm(const float *part, int S, const float *src, float *x, const float *w, float eps, float *xn, int M,
                       int H, hipStream_t st);
// h[m][c] = SiLU(gate) * up from [gate | up] partials of width 2F.
void launch_swiglu(const float *part, int S, int M, int F, float *h, hipStream_t st);
// y[m][n] = act(sum_s part + bias) + residual (act: 0 none, 1 SiLU).
void launch_finish_linear(const float *part, int S, int M, int N, const float *bias, const float *residual, int act, float *y,
                          int ldy, hipStream_t st);

} // namespace pf
} // namespace navi_amd
