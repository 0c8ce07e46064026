// The Mamba-1 mixer's depthwise causal convolution on gfx950, the step before the scan
// in Hugging Face's MambaMixer (transformers modeling_mamba.py causal_conv1d_fn; the
// reference runs it upstream, python/arm_scan/patch.py patches only the scan):
//
//   y[b, d, t] = act(bias[d] + sum_{k < K} w[d, k] * x[b, d, t - (K-1) + k]),  x[t < 0] = 0
//
// x is any strided (batch, dim, len) view. The mixer hands over the first half of its
// in_proj output, (batch, len, 2*dim) storage, so channels are the contiguous axis.
// y is written (batch, dim, len) contiguous, the layout F.conv1d returns. The
// convolution is a transpose as well: a block stages a tile of kConvT + K - 1 steps x
// kConvD channels through LDS. It reads the tile along channels, the contiguous axis of
// such views, and writes along time.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "scan_common.h"
#include "scan_launch.h"

namespace armscan {

namespace {

constexpr int kConvD = 64;        // channels per tile
constexpr int kConvT = 64;        // steps per tile
constexpr int kConvMaxK = 8;      // widest filter served
constexpr int kConvThreads = 256;

__global__ void __launch_bounds__(kConvThreads) causal_conv_kernel(CausalConv p) {
  __shared__ float tile[(kConvT + kConvMaxK - 1) * (kConvD + 1)];  // [step][channel], padded
  const int K = p.width;
  const long long b = blockIdx.z;
  const int d0 = blockIdx.y * kConvD;
  const long long t0 = (long long)blockIdx.x * kConvT;
  const int rows = kConvT + K - 1;  // steps t0-(K-1) .. t0+kConvT-1
  const float* xb = p.x + b * p.xs[0];
  if (p.vec) {
    // unit channel stride, 16-byte aligned rows: four channels per load
    for (int e = threadIdx.x; e < rows * (kConvD / 4); e += kConvThreads) {
      const int r = e / (kConvD / 4), c = 4 * (e - r * (kConvD / 4));
      const long long t = t0 - (K - 1) + r;
      const int d = d0 + c;
      float4 v = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
      if (t >= 0 && t < p.len && d < p.dim)  // dim % 4 == 0: the piece is whole
        v = *reinterpret_cast<const float4*>(xb + d + t * p.xs[2]);
      float* row = tile + r * (kConvD + 1) + c;
      row[0] = v.x; row[1] = v.y; row[2] = v.z; row[3] = v.w;
    }
  } else {
    for (int e = threadIdx.x; e < rows * kConvD; e += kConvThreads) {
      const int r = e / kConvD, c = e - r * kConvD;
      const long long t = t0 - (K - 1) + r;
      const int d = d0 + c;
      float v = 0.0f;
      if (t >= 0 && t < p.len && d < p.dim) v = xb[(long long)d * p.xs[1] + t * p.xs[2]];
      tile[r * (kConvD + 1) + c] = v;
    }
  }
  __syncthreads();
  if (p.out_tm) {
    // (batch, len, dim) storage: consecutive lanes take consecutive channels, and a
    // thread keeps one channel (kConvThreads is a multiple of kConvD), whose taps and
    // bias it loads once
    static_assert(kConvThreads % kConvD == 0, "a thread keeps its channel");
    const int c = threadIdx.x % kConvD;
    const int d = d0 + c;
    if (d >= p.dim) return;  // no barrier follows
    float wr[kConvMaxK];
#pragma unroll
    for (int k = 0; k < kConvMaxK; ++k) wr[k] = k < K ? p.w[(long long)d * K + k] : 0.0f;
    const float bv = p.bias ? p.bias[d] : 0.0f;
    for (int r = threadIdx.x / kConvD; r < kConvT; r += kConvThreads / kConvD) {
      const long long t = t0 + r;
      if (t >= p.len) break;
      float acc = bv;
#pragma unroll
      for (int k = 0; k < kConvMaxK; ++k)
        if (k < K) acc = fmaf(wr[k], tile[(r + k) * (kConvD + 1) + c], acc);
      if (p.silu) acc = silu_fast(acc);
      p.out[(b * p.len + t) * p.dim + d] = acc;
    }
    return;
  }
  // (batch, dim, len): a thread keeps one step (kConvThreads is a multiple of kConvT)
  // and walks the channels, each wave on one channel, so taps and bias are uniform
  static_assert(kConvThreads % kConvT == 0, "a thread keeps its step");
  const int r = threadIdx.x % kConvT;
  const long long t = t0 + r;
  if (t >= p.len) return;  // no barrier follows
  for (int c = threadIdx.x / kConvT; c < kConvD; c += kConvThreads / kConvT) {
    const int d = d0 + c;
    if (d >= p.dim) break;
    float acc = p.bias ? p.bias[d] : 0.0f;
#pragma unroll
    for (int k = 0; k < kConvMaxK; ++k)
      if (k < K) acc = fmaf(p.w[(long long)d * K + k], tile[(r + k) * (kConvD + 1) + c], acc);
    if (p.silu) acc = silu_fast(acc);
    p.out[(b * p.dim + d) * p.len + t] = acc;
  }
}

// One decode step: thread (b, d) shifts its window of the conv state left by one,
// appends the new input and writes act(bias + w . window).
__global__ void __launch_bounds__(kConvThreads) causal_conv_step_kernel(CausalConvStep p) {
  const long long i = (long long)blockIdx.x * kConvThreads + threadIdx.x;  // b * dim + d
  if (i >= (long long)p.batch * p.dim) return;
  const long long b = i / p.dim, d = i - b * p.dim;
  float* s = p.state + i * p.width;
  const float* w = p.w + d * p.width;
  const float x = p.x[b * p.xs[0] + d * p.xs[1]];
  float acc = p.bias ? p.bias[d] : 0.0f;
  for (int k = 0; k < p.width; ++k) {
    const float v = k + 1 < p.width ? s[k + 1] : x;
    s[k] = v;
    acc = fmaf(w[k], v, acc);
  }
  if (p.silu) acc = silu(acc);
  p.out[i] = acc;
}

}  // namespace

hipError_t causal_conv1d_step(const CausalConvStep& p, hipStream_t st) {
  const long long rows = (long long)p.batch * p.dim;
  const long long blocks = (rows + kConvThreads - 1) / kConvThreads;
  if (blocks <= 0 || blocks > 0x7fffffffLL || p.width < 1) return hipErrorInvalidValue;
  hipLaunchKernelGGL(causal_conv_step_kernel, dim3((unsigned)blocks), dim3(kConvThreads), 0,
                     st, p);
  return hipGetLastError();
}

hipError_t causal_conv1d(const CausalConv& p, hipStream_t st) {
  if (p.width < 1 || p.width > kConvMaxK || p.batch < 1 || p.dim < 1 || p.len < 1)
    return hipErrorInvalidValue;
  const long long tb = (p.len + kConvT - 1) / kConvT;
  if (tb > 0x7fffffffLL || p.batch > 65535 || (p.dim + kConvD - 1) / kConvD > 65535)
    return hipErrorInvalidValue;
  const dim3 grid((unsigned)tb, (unsigned)((p.dim + kConvD - 1) / kConvD), (unsigned)p.batch);
  CausalConv k = p;
  k.vec = p.xs[1] == 1 && p.dim % 4 == 0 && p.xs[0] % 4 == 0 && p.xs[2] % 4 == 0 &&
          ((uintptr_t)p.x & 15u) == 0;
  hipLaunchKernelGGL(causal_conv_kernel, grid, dim3(kConvThreads), 0, st, k);
  return hipGetLastError();
}

}  // namespace armscan
