// Mamba-3 RoPE angle pre-pass on gfx950 (python/arm_scan/mamba3.py:41-89):
//
//   theta[b, t, h, u] = sum_{s <= t} tanh(angle[b, s, h, u]) * pi * dt[b, h, s]
//   cos, sin = cos(theta), sin(theta)      (b, l, h, half); pairs u >= r: 1, 0
//
// in one pass: angles and dt read once, cos and sin written once (the torch
// formulation runs tanh, two products, the cumsum, cos, sin and the padding as
// separate passes over the tensor).
//
// A block owns one 16-byte piece of pairs, u = 4*u4 .. 4*u4+3, of one (batch, head)
// and walks the sequence in tiles of 1024 steps: each of its 256 threads sums the
// increments of 4 consecutive steps, the block scans those sums (a wave scan, then
// the four wave totals through LDS), and every thread writes cos/sin of its 4 steps.
// The angle reached at the end of a tile carries into the next. A block whose
// pairs are all past r only writes the identity rotation.
//
// Block order: the 8 pieces of one 128-byte line of a (batch, step, head) row of
// cos/sin (pairs 32j .. 32j+31) come from 8 blocks on one XCD (block id mod 8),
// so that each line is assembled and written back by one L2.

#include <hip/hip_runtime.h>

#include <cstdint>

#include "scan_common.h"
#include "scan_launch.h"

namespace armscan {

namespace {

struct AngK {
  const float *ang, *dt;
  float *cos, *sin;
  int L, H, r, half;
  long long ngroups;  // line groups: (batch * heads) * ceil(half / 32)
  int vec;            // 16-byte pieces for angles (r % 4 == 0) and cos/sin (half % 4 == 0)
};

constexpr int kAngThreads = 256;
constexpr int kAngSteps = 4;  // consecutive steps per thread and tile

// tanh(a) = 1 - 2 / (1 + e^{2a}); saturates to +-1 through e^{2a} = inf or 0.
__device__ __forceinline__ float tanh_pp(float a) {
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + fexp(2.0f * a));
}

__device__ __forceinline__ float wave_inclusive_sum(float v, int lane) {
#pragma unroll
  for (int d = 1; d < 64; d <<= 1) {
    const float o = __shfl_up(v, d);
    if (lane >= d) v += o;
  }
  return v;
}

__global__ void __launch_bounds__(kAngThreads) m3_angles_kernel(AngK p) {
  const int x = blockIdx.x & 7;
  const long long k = blockIdx.x >> 3;
  const long long g = 8 * (k >> 3) + x;  // line group, on XCD x
  const int m = (int)(k & 7);            // piece within the line
  if (g >= p.ngroups) return;            // whole block: no barrier is reached
  const int gpr = (p.half + 31) / 32;
  const long long bh = g / gpr;          // batch * H + head
  const int u0 = 4 * ((int)(g % gpr) * 8 + m);
  if (u0 >= p.half) return;
  const long long b = bh / p.H, h = bh - b * p.H;
  const long long cstride = (long long)p.H * p.half;  // floats between steps
  float* cosp = p.cos + (b * p.L * p.H + h) * p.half + u0;
  float* sinp = p.sin + (b * p.L * p.H + h) * p.half + u0;
  const int tid = threadIdx.x;
  const int nu = p.half - u0 < 4 ? p.half - u0 : 4;  // pairs of this piece

  auto store = [&](long long t, const float (&c)[4], const float (&s)[4]) {
    if (p.vec) {
      *reinterpret_cast<float4*>(cosp + t * cstride) = make_float4(c[0], c[1], c[2], c[3]);
      *reinterpret_cast<float4*>(sinp + t * cstride) = make_float4(s[0], s[1], s[2], s[3]);
    } else {
      for (int e = 0; e < nu; ++e) {
        cosp[t * cstride + e] = c[e];
        sinp[t * cstride + e] = s[e];
      }
    }
  };

  if (u0 >= p.r) {  // no angle: the identity rotation
    const float one[4] = {1.0f, 1.0f, 1.0f, 1.0f}, zero[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (long long t = tid; t < p.L; t += kAngThreads) store(t, one, zero);
    return;
  }

  const float* angp = p.ang + (b * p.L * p.H + h) * p.r + u0;
  const long long astride = (long long)p.H * p.r;
  const float* dtp = p.dt + bh * p.L;
  const int na = p.r - u0 < 4 ? p.r - u0 : 4;  // pairs of this piece with an angle
  const int lane = tid & 63, wave = tid >> 6;
  __shared__ float wsum[kAngThreads / 64][4];

  float carry[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  for (long long t0 = 0; t0 < p.L; t0 += kAngThreads * kAngSteps) {
    const long long tb = t0 + (long long)tid * kAngSteps;
    float pre[kAngSteps][4];  // inclusive sums over the thread's steps
    float tot[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int j = 0; j < kAngSteps; ++j) {
      const long long t = tb + j;
      float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      float pdt = 0.0f;
      if (t < p.L) {
        pdt = 3.14159265358979f * dtp[t];
        if (p.vec) {
          const float4 v = *reinterpret_cast<const float4*>(angp + t * astride);
          a[0] = v.x; a[1] = v.y; a[2] = v.z; a[3] = v.w;
        } else {
          for (int e = 0; e < na; ++e) a[e] = angp[t * astride + e];
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        tot[e] += tanh_pp(a[e]) * pdt;  // pairs past r: a = 0, so 0
        pre[j][e] = tot[e];
      }
    }
    // exclusive prefix of the thread sums over the block, plus the carry
    float base[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float incl = wave_inclusive_sum(tot[e], lane);
      if (lane == 63) wsum[wave][e] = incl;
      base[e] = incl - tot[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float before = 0.0f, all = 0.0f;
#pragma unroll
      for (int w = 0; w < kAngThreads / 64; ++w) {
        const float v = wsum[w][e];
        if (w < wave) before += v;
        all += v;
      }
      base[e] += carry[e] + before;
      carry[e] += all;
    }
    __syncthreads();  // wsum is rewritten by the next tile
#pragma unroll
    for (int j = 0; j < kAngSteps; ++j) {
      const long long t = tb + j;
      if (t >= p.L) break;
      float c[4], s[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // cos/sin of revolutions, theta / 2pi reduced to [-1/2, 1/2]
        const float rev = (base[e] + pre[j][e]) * 0.15915494309189535f;
        const float f = rev - __builtin_rintf(rev);
        c[e] = __builtin_amdgcn_cosf(f);
        s[e] = __builtin_amdgcn_sinf(f);
      }
      store(t, c, s);
    }
  }
}

}  // namespace

hipError_t m3_angles_to_cos_sin(const float* angles, const float* dt, size_t batch,
                                size_t len, size_t heads, size_t r, size_t half, float* cos,
                                float* sin, hipStream_t st) {
  AngK k{};
  k.ang = angles; k.dt = dt; k.cos = cos; k.sin = sin;
  k.L = (int)len; k.H = (int)heads; k.r = (int)r; k.half = (int)half;
  k.ngroups = (long long)(batch * heads) * (long long)((half + 31) / 32);
  const bool a16 = ((uintptr_t)angles & 15u) == 0 && ((uintptr_t)cos & 15u) == 0 &&
                   ((uintptr_t)sin & 15u) == 0;
  k.vec = a16 && r % 4 == 0 && half % 4 == 0;
  const long long blocks = 64 * ((k.ngroups + 7) / 8);
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  hipLaunchKernelGGL(m3_angles_kernel, dim3((unsigned)blocks), dim3(kAngThreads), 0, st, k);
  return hipGetLastError();
}

}  // namespace armscan
