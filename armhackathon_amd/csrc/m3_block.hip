// The Mamba-3 mixer's front-end on gfx950 (apps/mamba3_lm/block.py:146-178): what
// sits between in_proj and the scan, in one kernel over the projection
//
//   proj (b, l, row_stride), columns [z | x | B | C | dd_dt | dd_A | trap | angles]
//   (block.py:113-118, the checkpoint's order)
//
//   dt   = softplus(dd_dt + dt_bias)                         -> (b, h, l)
//   adt  = min(-heavy_tail(dd_A), -A_floor) * dt              -> (b, h, l)
//          heavy_tail(x) = max(x, 0) + 1 / (1 - min(x, 0))    (block.py:52-62)
//   trap = trap, pre-sigmoid                                  -> (b, h, l)
//   k    = B * rsqrt(mean_n(B^2) + eps) * B_norm.weight       -> (b, l, r, g, n)
//   q    = C * rsqrt(mean_n(C^2) + eps) * C_norm.weight       (Q <- C, K <- B: block.py:187-197)
//
// z, x and the angles are not touched: the scan reads them in place from the
// projection by their strides (the angles with head stride 0, one set shared by every
// head as block.py:174 broadcasts them).
//
// A block takes kTok consecutive tokens of one batch row. The gates go through LDS, 32
// heads at a time, so that their head-major stores run along the sequence (kTok floats
// per head). The
// normalised rows of B and C (d_state floats each) take one wave each.

#include <hip/hip_runtime.h>

#include "scan_common.h"
#include "scan_launch.h"

namespace armscan {

namespace {

constexpr int kTok = 32;
constexpr int kHeadGroup = 32;  // heads per pass through LDS
constexpr int kFrontThreads = 256;

__global__ void __launch_bounds__(kFrontThreads) m3_frontend_kernel(M3Frontend p) {
  __shared__ float gl[3 * kHeadGroup * kTok];  // [3][head in group][token]: dt, adt, trap
  const int H = p.heads, L = p.len, n = p.d_state, rows = p.rank * p.groups;
  const long long b = blockIdx.y;
  const int t0 = blockIdx.x * kTok;
  const int ntok = L - t0 < kTok ? L - t0 : kTok;
  const float* base = p.proj + (b * L + t0) * p.row_stride;
  const int col_b = 2 * H * p.headdim, col_c = col_b + rows * n, col_g = col_c + rows * n;

  constexpr int G = kHeadGroup;
  for (int h0 = 0; h0 < H; h0 += G) {  // block-uniform
    const int nh = H - h0 < G ? H - h0 : G;
    for (int e = threadIdx.x; e < ntok * nh; e += kFrontThreads) {
      const int j = e / nh, hh = e - j * nh, h = h0 + hh;
      const float* g = base + (long long)j * p.row_stride + col_g;
      const float dt = softplus(g[h] + p.dt_bias[h]);
      const float x = g[H + h];
      const float heavy = fmaxf(x, 0.0f) + 1.0f / (1.0f - fminf(x, 0.0f));
      gl[hh * kTok + j] = dt;
      gl[(G + hh) * kTok + j] = fminf(-heavy, -p.a_floor) * dt;
      gl[(2 * G + hh) * kTok + j] = g[2 * H + h];
    }
    __syncthreads();
    for (int e = threadIdx.x; e < nh * ntok; e += kFrontThreads) {
      const int hh = e / ntok, j = e - hh * ntok;
      const long long o = (b * H + h0 + hh) * L + t0 + j;
      p.dt[o] = gl[hh * kTok + j];
      p.adt[o] = gl[(G + hh) * kTok + j];
      p.trap[o] = gl[(2 * G + hh) * kTok + j];
    }
    __syncthreads();  // gl is rewritten by the next group
  }

  // RMSNorm rows: (token j, B or C, row rr), one wave each
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int r = wave; r < 2 * rows * ntok; r += kFrontThreads / 64) {
    const int j = r / (2 * rows), rem = r - j * 2 * rows;
    const bool is_c = rem >= rows;
    const int rr = is_c ? rem - rows : rem;
    const float* src = base + (long long)j * p.row_stride + (is_c ? col_c : col_b) + rr * n;
    float ss = 0.0f;
    for (int e = lane; e < n; e += 64) ss = fmaf(src[e], src[e], ss);
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) ss += __shfl_xor(ss, d);
    const float rstd = 1.0f / sqrtf(ss / (float)n + p.eps);
    const float* w = is_c ? p.c_norm : p.b_norm;
    float* dst = (is_c ? p.q : p.k) + ((b * L + t0 + j) * rows + rr) * (long long)n;
    for (int e = lane; e < n; e += 64) dst[e] = src[e] * rstd * w[e];
  }
}

}  // namespace

hipError_t m3_frontend(const M3Frontend& p, hipStream_t st) {
  if (p.len <= 0 || p.batch <= 0 || p.heads <= 0) return hipErrorInvalidValue;
  const dim3 grid((unsigned)((p.len + kTok - 1) / kTok), (unsigned)p.batch);
  hipLaunchKernelGGL(m3_frontend_kernel, grid, dim3(kFrontThreads), 0, st, p);
  return hipGetLastError();
}

}  // namespace armscan
