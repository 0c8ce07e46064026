// Mamba-3 RoPE angle pre-pass on gfx950 (python/arm_scan/mamba3.py:41-89):
//
//   theta[b, t, h, u] = sum_{s <= t} tanh(angle[b, s, h, u]) * pi * dt[b, h, s]
//   cos, sin = cos(theta), sin(theta)      (b, l, h, half); pairs u >= r: 1, 0
//
// in one pass: angles and dt read once, cos and sin written once (the torch
// formulation runs tanh, two products, the cumsum, cos, sin and the padding as
// separate passes over the tensor).
//
// A block owns one 128-byte line of pairs (u = 32g .. 32g+31: 8 pieces of 4) of one
// (batch, head) over one segment of the sequence, walked in tiles of 128 steps.
// Thread (piece m = tid % 8, step lane sl = tid / 8) sums the increments of its 4
// consecutive steps; the block scans those sums over the step lanes (a shuffle scan
// over the 8 step lanes of a wave, then the wave totals through LDS) and every
// thread writes cos/sin of its steps. Each load and store instruction then covers
// 8 steps x 8 pieces, 8 whole lines. The angle reached at the end of a tile carries
// into the next. When the lines alone are too few to fill the chip, the sequence is
// cut into segments: a first kernel sums each segment's increments, and the block
// of segment s starts from the sum of the segments before it. Pieces whose pairs
// are all past r only write the identity rotation.
//
// Angles are summed in turns (theta / 2pi; an increment is tanh(angle) * dt / 2) and
// every carried sum is reduced to [-1/2, 1/2] turns, the period of cos/sin: a sum
// never grows, so each add rounds at ulp(1/2) turns, where a running theta in
// radians rounds at ulp(theta) (1.5e-5 rad near 225 rad, which one-signed angles
// reach over 4096 steps).

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
  long long nlines;  // (batch * heads) * ceil(half / 32)
  int vec;           // 16-byte pieces for angles (r % 4 == 0) and cos/sin (half % 4 == 0)
  long long ab, at, ah;  // element strides of the angles: batch, step, head
  int segs, seg_len;  // sequence segments per line, steps per segment (multiple of kTile)
  float* seg_tot;     // [nlines][segs][32]: the increments summed over each segment
};

constexpr int kAngThreads = 256;
constexpr int kPieces = 8;                         // pieces of 4 pairs per line
constexpr int kStepLanes = kAngThreads / kPieces;  // 32
constexpr int kAngSteps = 4;                       // consecutive steps per thread and tile
constexpr int kTile = kStepLanes * kAngSteps;      // 128 steps

// x turns reduced to [-1/2, 1/2] (exact: x - rint(x) is representable)
__device__ __forceinline__ float turns_mod1(float x) { return x - __builtin_rintf(x); }

// tanh(a) = 1 - 2 / (1 + e^{2a}); saturates to +-1 through e^{2a} = inf or 0.
__device__ __forceinline__ float tanh_pp(float a) {
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + fexp(2.0f * a));
}

// Where thread (piece m, step lane sl) of the block of `line` reads and writes.
struct AngLine {
  const float *angp, *dtp;
  float *cosp, *sinp;
  long long astride, cstride;
  int m, sl, nu, na;

  __device__ AngLine(const AngK& p, long long line) {
    const int gpr = (p.half + 31) / 32;
    const long long bh = line / gpr;  // batch * H + head
    m = threadIdx.x % kPieces;
    sl = threadIdx.x / kPieces;
    const int u0 = (int)(line % gpr) * 32 + 4 * m;  // the thread's piece of pairs
    const long long b = bh / p.H, h = bh - b * p.H;
    cstride = (long long)p.H * p.half;  // floats between steps
    cosp = p.cos + (b * p.L * p.H + h) * p.half + u0;
    sinp = p.sin + (b * p.L * p.H + h) * p.half + u0;
    nu = u0 >= p.half ? 0 : (p.half - u0 < 4 ? p.half - u0 : 4);  // pairs here
    na = u0 >= p.r ? 0 : (p.r - u0 < 4 ? p.r - u0 : 4);           // pairs with an angle
    angp = p.ang + b * p.ab + h * p.ah + u0;
    astride = p.at;
    dtp = p.dt + bh * p.L;
  }

  // the thread's increments tanh(angle) * dt / 2 (turns) of its steps of the tile at
  // t0, as inclusive sums in pre and their total in tot (0 past r and past L)
  __device__ __forceinline__ void tile_sums(const AngK& p, long long t0,
                                            float (&pre)[kAngSteps][4],
                                            float (&tot)[4]) const {
#pragma unroll
    for (int e = 0; e < 4; ++e) tot[e] = 0.0f;
#pragma unroll
    for (int j = 0; j < kAngSteps; ++j) {
      const long long t = t0 + (long long)sl * kAngSteps + j;
      float a[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      float hdt = 0.0f;
      if (t < p.L && na > 0) {
        hdt = 0.5f * dtp[t];  // pi * dt radians in turns (exact)
        if (p.vec) {
          const float4 v = *reinterpret_cast<const float4*>(angp + t * astride);
          a[0] = v.x; a[1] = v.y; a[2] = v.z; a[3] = v.w;
        } else {
          for (int e = 0; e < na; ++e) a[e] = angp[t * astride + e];
        }
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        tot[e] += tanh_pp(a[e]) * hdt;  // pairs past r: a = 0, so 0
        pre[j][e] = tot[e];
      }
    }
  }
};

// seg_tot of every (line, segment) whose line holds angles, but the last segment,
// whose sum no block reads (other blocks return at once, whole blocks).
__global__ void __launch_bounds__(kAngThreads) m3_angle_totals_kernel(AngK p) {
  const long long line = blockIdx.x / (p.segs - 1);
  const int seg = (int)(blockIdx.x - line * (p.segs - 1));
  const int gpr = (p.half + 31) / 32;
  if (line >= p.nlines || (int)(line % gpr) * 32 >= p.r) return;
  const AngLine ln(p, line);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ float wsum[kAngThreads / 64][kPieces][4];
  float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  const long long t_end = (long long)(seg + 1) * p.seg_len;  // below L: not the last
  for (long long t0 = (long long)seg * p.seg_len; t0 < t_end; t0 += kTile) {
    float pre[kAngSteps][4], tot[4];
    ln.tile_sums(p, t0, pre, tot);
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] = turns_mod1(acc[e] + tot[e]);
  }
#pragma unroll
  for (int e = 0; e < 4; ++e) {
#pragma unroll
    for (int d = kPieces; d < 64; d <<= 1) acc[e] = turns_mod1(acc[e] + __shfl_xor(acc[e], d));
    if (lane < kPieces) wsum[wave][ln.m][e] = acc[e];
  }
  __syncthreads();
  if (tid < kPieces) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float s = 0.0f;
#pragma unroll
      for (int w = 0; w < kAngThreads / 64; ++w) s = turns_mod1(s + wsum[w][tid][e]);
      p.seg_tot[(line * p.segs + seg) * 32 + 4 * tid + e] = turns_mod1(s);
    }
  }
}

__global__ void __launch_bounds__(kAngThreads) m3_angles_kernel(AngK p) {
  const long long line = blockIdx.x / p.segs;
  const int seg = (int)(blockIdx.x - line * p.segs);
  if (line >= p.nlines) return;  // whole block: no barrier is reached
  const AngLine ln(p, line);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  __shared__ float wsum[kAngThreads / 64][kPieces][4];

  auto store = [&](long long t, const float (&c)[4], const float (&s)[4]) {
    if (p.vec && ln.nu == 4) {
      *reinterpret_cast<float4*>(ln.cosp + t * ln.cstride) =
          make_float4(c[0], c[1], c[2], c[3]);
      *reinterpret_cast<float4*>(ln.sinp + t * ln.cstride) =
          make_float4(s[0], s[1], s[2], s[3]);
    } else {
      for (int e = 0; e < ln.nu; ++e) {
        ln.cosp[t * ln.cstride + e] = c[e];
        ln.sinp[t * ln.cstride + e] = s[e];
      }
    }
  };

  // the angle reached before the segment: the sums of the segments before it
  float carry[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (ln.na > 0) {
    for (int s = 0; s < seg; ++s) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        carry[e] = turns_mod1(carry[e] + p.seg_tot[(line * p.segs + s) * 32 + 4 * ln.m + e]);
    }
  }
  const long long t_end = (long long)(seg + 1) * p.seg_len;
  for (long long t0 = (long long)seg * p.seg_len; t0 < t_end && t0 < p.L; t0 += kTile) {
    const long long tb = t0 + (long long)ln.sl * kAngSteps;
    float pre[kAngSteps][4];  // inclusive sums over the thread's steps
    float tot[4];
    ln.tile_sums(p, t0, pre, tot);
    // exclusive prefix of the thread sums over the step lanes of the piece
    float base[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float incl = tot[e];
#pragma unroll
      for (int d = kPieces; d < 64; d <<= 1) {  // the wave's 8 step lanes, 8 lanes apart
        const float o = __shfl_up(incl, d);
        if (lane >= d) incl += o;
      }
      if (lane >= 64 - kPieces) wsum[wave][ln.m][e] = incl;  // the wave's total
      base[e] = incl - tot[e];
    }
    __syncthreads();
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      float before = 0.0f, all = 0.0f;
#pragma unroll
      for (int w = 0; w < kAngThreads / 64; ++w) {
        const float v = wsum[w][ln.m][e];
        if (w < wave) before += v;
        all += v;
      }
      base[e] += carry[e] + before;
      carry[e] = turns_mod1(carry[e] + all);
    }
    __syncthreads();  // wsum is rewritten by the next tile
    if (ln.nu == 0) continue;
#pragma unroll
    for (int j = 0; j < kAngSteps; ++j) {
      const long long t = tb + j;
      if (t >= p.L || t >= t_end) break;
      float c[4], s[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // cos/sin of turns reduced to [-1/2, 1/2]
        const float f = turns_mod1(base[e] + pre[j][e]);
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
                                float* sin, hipStream_t st, const long long* ang_strides) {
  AngK k{};
  k.ang = angles; k.dt = dt; k.cos = cos; k.sin = sin;
  k.L = (int)len; k.H = (int)heads; k.r = (int)r; k.half = (int)half;
  k.nlines = (long long)(batch * heads) * (long long)((half + 31) / 32);
  const bool a16 = ((uintptr_t)angles & 15u) == 0 && ((uintptr_t)cos & 15u) == 0 &&
                   ((uintptr_t)sin & 15u) == 0;
  if (ang_strides) {
    k.ab = ang_strides[0]; k.at = ang_strides[1]; k.ah = ang_strides[2];
  } else {
    k.ah = (long long)r;
    k.at = (long long)(heads * r);
    k.ab = (long long)(len * heads * r);
  }
  k.vec = a16 && r % 4 == 0 && half % 4 == 0 && k.ab % 4 == 0 && k.at % 4 == 0 &&
          k.ah % 4 == 0;
  if (len == 0 || k.nlines == 0) return hipSuccess;
  // segments: enough blocks to fill the chip a few times over
  const long long tiles = ((long long)len + kTile - 1) / kTile;
  long long segs = k.nlines > 0 ? (2048 + k.nlines - 1) / k.nlines : 1;
  if (segs > tiles) segs = tiles;
  if (segs < 1) segs = 1;
  const long long seg_tiles = (tiles + segs - 1) / segs;
  k.seg_len = (int)(seg_tiles * kTile);
  k.segs = (int)((tiles + seg_tiles - 1) / seg_tiles);
  if (k.segs < 1) k.segs = 1;
  const long long blocks = k.nlines * k.segs;
  if (blocks > 0x7fffffffLL) return hipErrorInvalidValue;
  if (k.segs > 1) {
    hipError_t e = stream_alloc((void**)&k.seg_tot, (size_t)blocks * 32 * sizeof(float), st);
    if (e != hipSuccess) return e;
    hipLaunchKernelGGL(m3_angle_totals_kernel, dim3((unsigned)(k.nlines * (k.segs - 1))),
                       dim3(kAngThreads), 0, st, k);
  }
  hipLaunchKernelGGL(m3_angles_kernel, dim3((unsigned)blocks), dim3(kAngThreads), 0, st, k);
  hipError_t e = hipGetLastError();
  if (k.segs > 1) {
    const hipError_t ef = hipFreeAsync(k.seg_tot, st);
    if (e == hipSuccess) e = ef;
  }
  return e;
}

}  // namespace armscan
