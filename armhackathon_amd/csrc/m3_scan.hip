// Mamba-3 SISO and rank-r MIMO scan on MI355X (gfx950).
//
// Semantics (kernel/arm-scan-core/src/mamba3/mod.rs:17-33, mamba3/scalar.rs:50-196,
// mamba3/mimo.rs:98-284), per (batch, head) with a (dv, dqk) state S:
//   lam = sigmoid(trap_t); gamma = dt_t lam; alpha = exp(adt_t)
//   scale = gamma + dt_nxt (1 - sigmoid(trap_nxt)), nxt = t+1 forward / t-1 reverse,
//           0 at the last step of the traversal
//   SISO: q, k = interleaved-RoPE(q + q_bias, k + k_bias)
//         y = alpha (q . S^T) + (D + gamma q.k) v ;  S = alpha S + scale v k^T
//         out = y silu(z); last_bx = scale k at the final step
//   MIMO: q_r, k_r = split-halves-RoPE(...); x_r = psi_r * v
//         acc_r = alpha q_r . S^T + gamma sum_b (q_r . k_b) x_b + D x_r
//         S = alpha S + scale sum_r x_r k_r^T
//         out = sum_r phi_r silu(z zeta_r) acc_r   (or sum_r phi_r acc_r without z)
//
// This kernel walks the sequence step by step with the state resident in LDS,
// one workgroup per (batch, head); every step is three barrier-separated
// phases: rotate q/k + gates, the q.S and Gram contractions, then the state
// update and the output.

#include <hip/hip_runtime.h>

#include "scan_common.h"
#include <cstdint>

#include "scan_launch.h"

namespace armscan {

namespace {

constexpr int kM3Threads = 256;
constexpr size_t kM3MaxLdsFloats = 15 * 1024;  // 60 KB

struct M3Args {
  const float *q, *k, *v, *adt, *dt, *trap, *qb, *kb, *cos, *sin, *D, *z, *psi, *zeta, *phi;
  float *out, *last_state, *last_bx;
  int heads, dv, dqk, len, rank, groups, reverse, mimo, out_tm, accumulate;
  long long vb, vt, zb, zt;  // element strides of v and z: batch, step
};

__global__ void __launch_bounds__(kM3Threads) m3_seq_kernel(M3Args p) {
  extern __shared__ float sm[];
  const int dv = p.dv, dqk = p.dqk, R = p.rank, half = dqk / 2, L = p.len;
  const int SP = dqk + 1;  // padded state row
  float* S = sm;
  float* qr = S + dv * SP;
  float* kr = qr + R * dqk;
  float* xs = kr + R * dqk;
  float* acc = xs + R * dv;
  float* gram = acc + R * dv;
  float* gts = gram + R * R;  // gamma, scale, alpha

  const int tid = threadIdx.x;
  const int bh = blockIdx.x;
  const int bi = bh / p.heads, h = bh - bi * p.heads;
  const int grp = h / (p.heads / p.groups);
  const long long gate_base = (long long)bh * L;
  const float dskip = p.D ? p.D[h] : 0.0f;
  // head-major (b, h, l, dv), or time-major (b, l, h, dv)
  float* orow = p.out_tm ? p.out + ((long long)bi * L * p.heads + h) * dv
                         : p.out + (long long)bh * L * dv;
  const long long ostep = p.out_tm ? (long long)p.heads * dv : dv;

  for (int e = tid; e < dv * SP; e += kM3Threads) S[e] = 0.0f;
  __syncthreads();

  for (int i = 0; i < L; ++i) {
    const int t = p.reverse ? L - 1 - i : i;
    // ---- phase 1: rotate q/k, project v, gates
    const long long cs_off = (((long long)bi * L + t) * p.heads + h) * half;
    for (int e = tid; e < R * dqk; e += kM3Threads) {
      const int rr = e / dqk, j = e - rr * dqk;
      const long long qo = ((((long long)bi * L + t) * R + rr) * p.groups + grp) * dqk;
      const float* qb = p.qb + ((long long)h * R + rr) * dqk;
      const float* kb = p.kb + ((long long)h * R + rr) * dqk;
      int j0, j1, pi;
      if (!p.mimo) {  // interleaved pairs (2i, 2i+1): mamba3/scalar.rs:40-48
        pi = j >> 1; j0 = 2 * pi; j1 = j0 + 1;
      } else {        // split halves (i, i + dqk/2): mimo.rs:83-96
        pi = j < half ? j : j - half; j0 = pi; j1 = pi + half;
      }
      const float c = p.cos[cs_off + pi], s = p.sin[cs_off + pi];
      const float qa = p.q[qo + j0] + qb[j0], qc = p.q[qo + j1] + qb[j1];
      const float ka = p.k[qo + j0] + kb[j0], kc = p.k[qo + j1] + kb[j1];
      const bool first = (j == j0);
      qr[e] = first ? (qa * c - qc * s) : (qa * s + qc * c);
      kr[e] = first ? (ka * c - kc * s) : (ka * s + kc * c);
    }
    const long long v_off = (long long)bi * p.vb + (long long)t * p.vt + (long long)h * dv;
    const long long z_off = (long long)bi * p.zb + (long long)t * p.zt + (long long)h * dv;
    for (int e = tid; e < R * dv; e += kM3Threads) {
      const int rr = e / dv, pp = e - rr * dv;
      const float vv = p.v[v_off + pp];
      xs[e] = p.mimo ? p.psi[((long long)h * R + rr) * dv + pp] * vv : vv;
    }
    if (tid == 0) {
      const long long g = gate_base + t;
      const float lam = sigmoid(p.trap[g]);
      const float gamma = p.dt[g] * lam;
      const bool has_nxt = p.reverse ? (i + 1 < L) : (t + 1 < L);
      const long long nx = p.reverse ? g - 1 : g + 1;
      const float shifted = has_nxt ? p.dt[nx] * (1.0f - sigmoid(p.trap[nx])) : 0.0f;
      gts[0] = gamma;
      gts[1] = gamma + shifted;
      gts[2] = fexp(p.adt[g]);
    }
    __syncthreads();
    // ---- phase 2: Gram matrix and q_r . S_p (state before this step)
    for (int e = tid; e < R * R; e += kM3Threads) {
      const int a = e / R, b = e - a * R;
      float sum = 0.0f;
      for (int j = 0; j < dqk; ++j) sum = fmaf(qr[a * dqk + j], kr[b * dqk + j], sum);
      gram[e] = sum;
    }
    for (int e = tid; e < R * dv; e += kM3Threads) {
      const int rr = e / dv, pp = e - rr * dv;
      const float* qrow = qr + rr * dqk;
      const float* srow = S + pp * SP;
      float sum = 0.0f;
      for (int j = 0; j < dqk; ++j) sum = fmaf(qrow[j], srow[j], sum);
      acc[e] = sum;
    }
    __syncthreads();
    // ---- phase 3: state update and output
    const float gamma = gts[0], scale = gts[1], alpha = gts[2];
    for (int e = tid; e < dv * dqk; e += kM3Threads) {
      const int pp = e / dqk, j = e - pp * dqk;
      float upd = 0.0f;
      for (int rr = 0; rr < R; ++rr) upd = fmaf(xs[rr * dv + pp], kr[rr * dqk + j], upd);
      float* sp = S + pp * SP + j;
      *sp = fmaf(alpha, *sp, scale * upd);
    }
    float* dst = orow + (long long)t * ostep;
    for (int pp = tid; pp < dv; pp += kM3Threads) {
      float o;
      if (!p.mimo) {
        const float diag = p.accumulate ? 0.0f : dskip + gamma * gram[0];
        o = fmaf(alpha, acc[pp], diag * xs[pp]);
        if (p.z) o *= silu(p.z[z_off + pp]);
        if (p.accumulate) o += dst[pp];  // the other traversal's output
      } else {
        o = 0.0f;
        const float zz = p.z ? p.z[z_off + pp] : 0.0f;
        for (int rr = 0; rr < R; ++rr) {
          float dsum = 0.0f;
          for (int b = 0; b < R; ++b) dsum = fmaf(gram[rr * R + b], xs[b * dv + pp], dsum);
          const float ar = alpha * acc[rr * dv + pp] + gamma * dsum + dskip * xs[rr * dv + pp];
          const long long pj = ((long long)h * R + rr) * dv + pp;
          const float gate = p.z ? silu(zz * p.zeta[pj]) : 1.0f;
          o = fmaf(p.phi[pj] * gate, ar, o);
        }
      }
      dst[pp] = o;
    }
    __syncthreads();
  }
  if (p.last_state) {
    float* ls = p.last_state + (long long)bh * dv * dqk;
    for (int e = tid; e < dv * dqk; e += kM3Threads) {
      const int pp = e / dqk, j = e - pp * dqk;
      ls[e] = S[pp * SP + j];
    }
  }
  if (p.last_bx) {
    const float scale = gts[1];
    for (int j = tid; j < dqk; j += kM3Threads) p.last_bx[(long long)bh * dqk + j] = scale * kr[j];
  }
}

size_t lds_floats(size_t dv, size_t dqk, size_t r) {
  return dv * (dqk + 1) + 2 * r * dqk + 2 * r * dv + r * r + 4;
}

}  // namespace

size_t m3_max_state() { return kM3MaxLdsFloats; }

static bool aligned16(const void* q) { return q == nullptr || ((uintptr_t)q & 15u) == 0; }

namespace {
bool m3_aligned(const M3Problem& pr) {
  // 16-byte pieces at every (batch, step, head) row start, strides included
  const bool strides4 = pr.v_strides[0] % 4 == 0 && pr.v_strides[1] % 4 == 0 &&
                        pr.z_strides[0] % 4 == 0 && pr.z_strides[1] % 4 == 0 &&
                        (pr.angles == nullptr ||
                         (pr.ang_strides[0] % 4 == 0 && pr.ang_strides[1] % 4 == 0 &&
                          pr.ang_strides[2] % 4 == 0));
  return strides4 && aligned16(pr.q) && aligned16(pr.k) && aligned16(pr.q_bias) &&
         aligned16(pr.k_bias) && aligned16(pr.cos) && aligned16(pr.sin) &&
         aligned16(pr.angles) && aligned16(pr.v) && aligned16(pr.z) &&
         aligned16(pr.last_state) && aligned16(pr.last_bx);
}
}  // namespace

bool m3_angles_supported(const M3Problem& pr, const char** why) {
  auto no = [&](const char* w) {
    if (why) *why = w;
    return false;
  };
  if (pr.reverse) return no("fused angles are forward only (theta is a forward cumsum)");
  if (pr.n_angles == 0 || pr.n_angles % 4 || pr.n_angles > pr.dqk / 2)
    return no("fused angles need n_angles a positive multiple of 4, at most dqk/2");
  if (!m3_aligned(pr)) return no("fused angles need 16-byte aligned inputs");
  if (!m3_chunk_supported(pr)) return no("fused angles need the chunked kernel's shapes");
  if (pr.len * pr.heads * pr.n_angles >= ((size_t)1 << 30))
    return no("angles span too large for 32-bit offsets");
  return true;
}

hipError_t m3_scan(const M3Problem& pr, hipStream_t st) {
  if (pr.accumulate && (pr.psi != nullptr || pr.rank != 1 || pr.angles))
    return hipErrorInvalidValue;  // the non-causal sum is defined for SISO on cos/sin
  if (pr.angles) {
    if (!m3_angles_supported(pr, nullptr)) return hipErrorInvalidValue;
    return m3_scan_chunked(pr, st);
  }
  if (m3_aligned(pr) && m3_chunk_supported(pr)) return m3_scan_chunked(pr, st);
  return m3_scan_sequential(pr, st);
}

hipError_t m3_scan_sequential(const M3Problem& pr, hipStream_t st) {
  const size_t fl = lds_floats(pr.dv, pr.dqk, pr.rank);
  if (fl > kM3MaxLdsFloats) return hipErrorInvalidValue;
  M3Args a{};
  a.q = pr.q; a.k = pr.k; a.v = pr.v; a.adt = pr.adt; a.dt = pr.dt; a.trap = pr.trap;
  a.qb = pr.q_bias; a.kb = pr.k_bias; a.cos = pr.cos; a.sin = pr.sin; a.D = pr.D; a.z = pr.z;
  a.psi = pr.psi; a.zeta = pr.zeta; a.phi = pr.phi;
  a.out = pr.out; a.last_state = pr.last_state; a.last_bx = pr.last_bx;
  a.heads = (int)pr.heads; a.dv = (int)pr.dv; a.dqk = (int)pr.dqk; a.len = (int)pr.len;
  a.rank = (int)pr.rank; a.groups = (int)pr.groups; a.reverse = pr.reverse;
  a.mimo = pr.psi != nullptr;
  a.out_tm = pr.out_time_major;
  a.accumulate = pr.accumulate;
  a.vb = pr.v_strides[0]; a.vt = pr.v_strides[1];
  a.zb = pr.z_strides[0]; a.zt = pr.z_strides[1];
  const unsigned blocks = (unsigned)(pr.batch * pr.heads);
  hipLaunchKernelGGL(m3_seq_kernel, dim3(blocks), dim3(kM3Threads), fl * sizeof(float), st, a);
  return hipGetLastError();
}

}  // namespace armscan
