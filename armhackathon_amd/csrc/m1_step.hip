// Mamba-1 decode: one step of the selective scan with the recurrent state updated
// in place, the single-token path of a generation loop (transformers
// modeling_mamba.py mamba_selective_state_update; the reference leaves it to upstream,
// README.md:320-322). Per (batch, channel) and state n:
//
//   dt = softplus(dt + bias) (when asked);  h_n <- exp(dt A_n) h_n + dt B_n x
//   y = sum_n C_n h_n + D x ;  y *= silu(z)
//
// the one-step case of scalar::scan (kernel/arm-scan-core/src/scalar.rs:11-89) with
// h0 = last_state = the state. One thread per (batch, channel) row: it reads and
// rewrites its state row and writes one output. The per-row inputs are given by
// strides, as a decoder hands them over (views of its projections); the work is
// a few hundred bytes per row, so what counts is that it is one launch.

#include <hip/hip_runtime.h>

#include "scan_common.h"
#include "scan_launch.h"

namespace armscan {

namespace {

constexpr int kStepThreads = 256;

__global__ void __launch_bounds__(kStepThreads) m1_step_kernel(M1Step p) {
  const long long i = (long long)blockIdx.x * kStepThreads + threadIdx.x;  // b * dim + d
  if (i >= (long long)p.batch * p.dim) return;
  const long long b = i / p.dim, d = i - b * p.dim;
  const float x = p.x[b * p.xs[0] + d * p.xs[1]];
  float dt = p.dt[b * p.dts[0] + d * p.dts[1]] + (p.bias ? p.bias[d] : 0.0f);
  if (p.softplus) dt = softplus(dt);
  float* h = p.state + i * p.N;
  const float* A = p.A + d * p.N;
  const float* B = p.B + b * p.Bs[0];
  const float* C = p.C + b * p.Cs[0];
  const float dx = dt * x;
  float y = 0.0f;
  for (int n = 0; n < p.N; ++n) {
    const float hn = fmaf(fexp(dt * A[n]), h[n], dx * B[n * p.Bs[1]]);
    h[n] = hn;
    y = fmaf(C[n * p.Cs[1]], hn, y);
  }
  if (p.D) y = fmaf(p.D[d], x, y);
  if (p.z) y *= silu(p.z[b * p.zs[0] + d * p.zs[1]]);
  p.out[i] = y;
}

}  // namespace

hipError_t m1_step(const M1Step& p, hipStream_t st) {
  const long long rows = (long long)p.batch * p.dim;
  const long long blocks = (rows + kStepThreads - 1) / kStepThreads;
  if (blocks <= 0 || blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(m1_step_kernel, dim3((unsigned)blocks), dim3(kStepThreads), 0, st, p);
  return hipGetLastError();
}

}  // namespace armscan
