// Device helpers shared by the Mamba-1 and Mamba-3 kernels (gfx950 / CDNA4).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace armscan {

constexpr float kLog2e = 1.4426950408889634f;
constexpr float kLn2 = 0.6931471805599453f;

// ------------------------------------------------------------------ math
// v_exp_f32 / v_log_f32: the hardware base-2 transcendentals.
__device__ __forceinline__ float ex2(float x) { return __builtin_amdgcn_exp2f(x); }
__device__ __forceinline__ float lg2(float x) { return __builtin_amdgcn_logf(x); }
__device__ __forceinline__ float fexp(float x) { return ex2(x * kLog2e); }

// log1p(e) for e >= 0, accurate for small e: log1p(e) = log(u) * e / (u - 1)
// with u = 1 + e (Goldberg, "What Every Computer Scientist Should Know About
// Floating-Point Arithmetic", ACM Computing Surveys 1991, Theorem 4). The
// rounding error of u cancels between log(u) and u - 1.
__device__ __forceinline__ float log1p_pos(float e) {
  const float u = 1.0f + e;
  const float d = u - 1.0f;
  return d == 0.0f ? e : (lg2(u) * kLn2) * (e / d);
}

// softplus with the reference's threshold: identity above 20 (float.rs:31-37).
__device__ __forceinline__ float softplus(float x) {
  return x > 20.0f ? x : log1p_pos(fexp(x));
}
// silu(x) = x / (1 + e^-x) (float.rs:41-43).
__device__ __forceinline__ float silu(float x) { return x / (1.0f + fexp(-x)); }
// The same with the hardware reciprocal (v_rcp_f32, 1 ulp) in place of the
// IEEE division: the hot-loop epilogues use this one.
__device__ __forceinline__ float silu_fast(float x) {
  return x * __builtin_amdgcn_rcpf(1.0f + fexp(-x));
}
// softplus for the hot loops, one transcendental fewer than the division form:
// with u = fl(1 + e) the rounding error r = (1 + e) - u equals e - (u - 1) exactly
// for u < 2 (u - 1 and then e - (u - 1) are exact by Sterbenz's lemma), and
// log1p(e) = log(u) + log1p(r/u), where log1p(r/u) = r to within e * 2^-24 of the
// result (|r| <= 2^-24). For u >= 2, r/u is below 2^-24 of log(u) and is dropped.
// e below 2^-24 gives u = 1, log(u) = 0 and the result e exactly.
__device__ __forceinline__ float softplus_fast(float x) {
  if (x > 20.0f) return x;
  const float e = fexp(x);
  const float u = 1.0f + e;
  const float r = e - (u - 1.0f);
  return fmaf(lg2(u), kLn2, u < 2.0f ? r : 0.0f);
}
// sigmoid evaluated on the non-positive branch (float.rs:52-59).
__device__ __forceinline__ float sigmoid(float x) {
  if (x >= 0.0f) return 1.0f / (1.0f + fexp(-x));
  const float e = fexp(x);
  return e / (1.0f + e);
}

// ------------------------------------------------------------------ wave64 DPP
// update_dpp(old, src): lanes whose DPP source is out of range, or whose row is
// masked off, keep `old` — used below to inject the scan identity.
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ float dpp(float old, float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(__float_as_int(old), __float_as_int(v),
                                                      CTRL, ROW_MASK, 0xF, false));
}
constexpr int kRowShl1 = 0x101, kRowShl2 = 0x102, kRowShl4 = 0x104, kRowShl8 = 0x108;
constexpr int kRowShr1 = 0x111, kRowShr2 = 0x112, kRowShr4 = 0x114, kRowShr8 = 0x118;
constexpr int kWaveShl1 = 0x130, kWaveShr1 = 0x138;
constexpr int kRowBcast15 = 0x142, kRowBcast31 = 0x143;
constexpr int kRowRor1 = 0x121, kWaveRor1 = 0x13C;
constexpr int kRowMirror = 0x140, kRowHalfMirror = 0x141;

__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Affine maps h -> a*h + b compose as (earlier, later) -> (a_e*a_l, a_l*b_e + b_l).
template <int CTRL, int ROW_MASK>
__device__ __forceinline__ void scan_step(float& a, float& b) {
  const float pa = dpp<CTRL, ROW_MASK>(1.0f, a);
  const float pb = dpp<CTRL, ROW_MASK>(0.0f, b);
  b = fmaf(a, pb, b);
  a = a * pa;
}

// Inclusive scan of affine pairs over lanes 0 -> 63 (Hillis-Steele within each
// row of 16 lanes, then the two row broadcasts across rows).
__device__ __forceinline__ void wave_scan_up(float& a, float& b) {
  scan_step<kRowShr1, 0xF>(a, b);
  scan_step<kRowShr2, 0xF>(a, b);
  scan_step<kRowShr4, 0xF>(a, b);
  scan_step<kRowShr8, 0xF>(a, b);
  scan_step<kRowBcast15, 0xA>(a, b);
  scan_step<kRowBcast31, 0xC>(a, b);
}

// Inclusive scan over lanes 63 -> 0 (suffix scan): within rows via row_shl,
// across rows via the row heads read into uniform registers.
__device__ __forceinline__ void wave_scan_down(float& a, float& b, int lane) {
  scan_step<kRowShl1, 0xF>(a, b);
  scan_step<kRowShl2, 0xF>(a, b);
  scan_step<kRowShl4, 0xF>(a, b);
  scan_step<kRowShl8, 0xF>(a, b);
  const float a1 = readlane(a, 16), b1 = readlane(b, 16);
  const float a2 = readlane(a, 32), b2 = readlane(b, 32);
  const float a3 = readlane(a, 48), b3 = readlane(b, 48);
  const int row = lane >> 4;
  float ia = 1.0f, ib = 0.0f;
  if (row <= 2) { ia = a3; ib = b3; }
  if (row <= 1) { ib = fmaf(a2, ib, b2); ia = ia * a2; }
  if (row == 0) { ib = fmaf(a1, ib, b1); ia = ia * a1; }
  b = fmaf(a, ib, b);
  a = a * ia;
}

}  // namespace armscan
