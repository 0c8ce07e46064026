// Mamba-3 SISO and rank-r MIMO scan on MI355X (gfx950): the chunked dual form on
// fp32 MFMA (v_mfma_f32_16x16x4f32).
//
// Per (batch, head) with a (dv x dqk) state S, the recurrence of mamba3/scalar.rs:50-196
// and mamba3/mimo.rs:98-284 unrolls, over a chunk of consecutive rows with
// cumulative log-decay c (c_i = sum of adt over the chunk's steps up to row i's),
// into
//   Y = (M o Q K^T) X + diag(e^c) Q S0^T + D X
//   S_end = e^{c_last} S0 + X^T diag(w) K,    w_s = e^{c_last - c_s} scale_s
//   M[i][s] = e^{c_i - c_s} scale_s  (step(s) < step(i)),  gamma_i (same step),  0 (later)
// A row is one (step, rank) pair; SISO is rank 1. A chunk holds 16 rows, so
// 16/R steps. The output of a step is the rank sum phi_r silu(z zeta_r) Y_r (MIMO)
// or Y silu(z) (SISO).
//
// Work decomposition: one block per (sequence, 16-row slice of dv) and one wave
// per 16-wide slice of dqk. Each wave keeps its 16x16 piece of S in MFMA
// registers and per chunk computes
//   its partial G^T = K Q^T over its dqk slice (4 MFMA),
//   its partial diag(e^c) Q S0^T (4 MFMA),
//   the update of its S piece (4 MFMA, through a K transpose in LDS);
// the partials meet in LDS and wave 0 adds the masked intra-chunk term (4 MFMA)
// and the epilogue. Every MFMA operand is used in the register layout the
// previous MFMA produced: the reduction index of each product is permuted so that
// lane l (row l%16, group j = l/16) always supplies element (l%16, 4j + r).
// The per-step gates come from a small pre-pass (m3_gates_kernel).

#include <hip/hip_runtime.h>

#include <cstdint>

#include "scan_common.h"
#include "scan_launch.h"

namespace armscan {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

struct M3Gates {
  // per (sequence, traversal step): {c, e^c, gamma, scale}; per step w; per chunk e^c_last
  f4* step;
  float* w;
  float* etot;
};

struct M3K {
  const float *q, *k, *v, *adt, *dt, *trap, *qb, *kb, *cos, *sin, *D, *z, *psi, *zeta, *phi;
  float *out, *last_state, *last_bx;
  M3Gates g;
  int batch, heads, dv, dqk, len, rank, groups, nparts, nchunks, steps_per_chunk, nseq;
};

// ---------------------------------------------------------------------------
// Gate pre-pass: one thread per (sequence, chunk). Traversal step g maps to memory
// t = g (forward) or L-1-g (reverse); the trapezoid's "next" step is traversal
// step g+1 (mamba3/scalar.rs:95-115), absent at the end of the traversal.
__global__ void __launch_bounds__(256) m3_gates_kernel(M3K p, int reverse) {
  const long long tid = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  const long long total = (long long)p.nseq * p.nchunks;
  if (tid >= total) return;
  const int seq = (int)(tid / p.nchunks);
  const int ch = (int)(tid - (long long)seq * p.nchunks);
  const int L = p.len, T = p.steps_per_chunk;
  const long long base = (long long)seq * L;  // gates are (b, h, l): seq = b*heads + h
  float c = 0.0f;
  float cs[16], sc[16];
  for (int i = 0; i < T; ++i) {
    const long long g = (long long)ch * T + i;
    float adt = 0.0f, gamma = 0.0f, scale = 0.0f;
    if (g < L) {
      const long long t = reverse ? L - 1 - g : g;
      adt = p.adt[base + t];
      const float lam = sigmoid(p.trap[base + t]);
      gamma = p.dt[base + t] * lam;
      scale = gamma;
      if (g + 1 < L) {
        const long long tn = reverse ? t - 1 : t + 1;
        scale = gamma + p.dt[base + tn] * (1.0f - sigmoid(p.trap[base + tn]));
      }
    }
    c += adt;
    cs[i] = c;
    sc[i] = scale;
    const long long o = (long long)seq * ((long long)p.nchunks * T) + (long long)ch * T + i;
    p.g.step[o] = f4{c, fexp(c), gamma, scale};
  }
  for (int i = 0; i < T; ++i) {
    const long long o = (long long)seq * ((long long)p.nchunks * T) + (long long)ch * T + i;
    p.g.w[o] = fexp(c - cs[i]) * sc[i];
  }
  p.g.etot[tid] = fexp(c);
}

// ---------------------------------------------------------------------------
// Rotated q/k for lane (row i, group j): the 4 columns n0 .. n0+3 of row i.
// SISO rotates interleaved pairs (2u, 2u+1) with angle u (mamba3/scalar.rs:40-48);
// MIMO rotates split halves (u, u + dqk/2) with angle u (mimo.rs:83-96).
template <bool MIMO>
__device__ __forceinline__ f4 rotated(const float* __restrict__ src, const float* __restrict__ bias,
                                      const float* __restrict__ cs, const float* __restrict__ sn,
                                      int n0, int dqk) {
  if (!MIMO) {
    const f4 x = *reinterpret_cast<const f4*>(src + n0) + *reinterpret_cast<const f4*>(bias + n0);
    const float2 c = *reinterpret_cast<const float2*>(cs + n0 / 2);
    const float2 s = *reinterpret_cast<const float2*>(sn + n0 / 2);
    return f4{x[0] * c.x - x[1] * s.x, x[0] * s.x + x[1] * c.x,
              x[2] * c.y - x[3] * s.y, x[2] * s.y + x[3] * c.y};
  }
  const int half = dqk / 2;
  const bool lo = n0 < half;
  const int u0 = lo ? n0 : n0 - half;  // angle index of column n0
  const int m0 = lo ? n0 + half : n0 - half;  // partner columns
  const f4 x = *reinterpret_cast<const f4*>(src + n0) + *reinterpret_cast<const f4*>(bias + n0);
  const f4 y = *reinterpret_cast<const f4*>(src + m0) + *reinterpret_cast<const f4*>(bias + m0);
  const f4 c = *reinterpret_cast<const f4*>(cs + u0);
  const f4 s = *reinterpret_cast<const f4*>(sn + u0);
  // low half: a*c - b*s with (a, b) = (x, y); high half: a*s + b*c with (a, b) = (y, x)
  return lo ? f4{x[0] * c[0] - y[0] * s[0], x[1] * c[1] - y[1] * s[1],
                 x[2] * c[2] - y[2] * s[2], x[3] * c[3] - y[3] * s[3]}
            : f4{y[0] * s[0] + x[0] * c[0], y[1] * s[1] + x[1] * c[1],
                 y[2] * s[2] + x[2] * c[2], y[3] * s[3] + x[3] * c[3]};
}

constexpr int kKtStride = 20;  // floats per row of the per-wave K transpose tile

template <int R, bool MIMO, bool REV>
__global__ void __launch_bounds__(1024) m3_chunk_kernel(M3K p) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int W = p.dqk / 16;  // waves per block
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15, lj = lane >> 4;
  // blocks of one sequence share an XCD (block id mod 8), and so its L2
  const int bx = blockIdx.x & 7, by = blockIdx.x >> 3;
  const int seq = (by / p.nparts) * 8 + bx;
  const int part = by - (by / p.nparts) * p.nparts;
  if (seq >= p.nseq) return;  // whole block exits: no barrier is reached by anyone
  const int bi = seq / p.heads, h = seq - bi * p.heads;
  const int grp = h / (p.heads / p.groups);
  const int L = p.len, dqk = p.dqk, dv = p.dv, H = p.heads;
  const int T = p.steps_per_chunk;  // 16 / R
  const int n0 = wave * 16 + 4 * lj;  // this lane's 4 columns of the wave's dqk slice
  const int pcol = part * 16 + li;    // this lane's state row (output column)
  const float dskip = p.D ? p.D[h] : 0.0f;

  float* part_buf = sm;                                   // [2][W][64][8]
  float* kt = sm + 2 * W * 64 * 8 + wave * 16 * kKtStride;  // [16][kKtStride] per wave

  // per-lane rank projections of the B-operand rows s = 4*lj + m (MIMO)
  float psi_m[4], zeta_r[4], phi_r[4];
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const int rk = (4 * lj + m) % R;
    psi_m[m] = MIMO ? p.psi[((long long)h * R + rk) * dv + pcol] : 1.0f;
    zeta_r[m] = (MIMO && p.z) ? p.zeta[((long long)h * R + rk) * dv + pcol] : 1.0f;
    phi_r[m] = MIMO ? p.phi[((long long)h * R + rk) * dv + pcol] : 1.0f;
  }

  f4 S = {0.0f, 0.0f, 0.0f, 0.0f};  // S[pcol][n0 .. n0+3]
  const long long gate_base = (long long)seq * p.nchunks * T;
  for (int ch = 0; ch < p.nchunks; ++ch) {
    // ---- this lane's row i = li: step, rank, gates, rotated q/k
    const int step_i = li / R, rank_i = li % R;
    const long long g_i = (long long)ch * T + step_i;
    const bool valid_i = g_i < L;
    const long long t_i = REV ? L - 1 - g_i : g_i;
    const f4 gi = p.g.step[gate_base + (long long)ch * T + step_i];  // {c, e, gamma, scale}
    f4 qr = {0.0f, 0.0f, 0.0f, 0.0f}, kr = qr;
    if (valid_i) {
      const long long row = (((long long)bi * L + t_i) * R + rank_i) * p.groups + grp;
      const long long cso = (((long long)bi * L + t_i) * H + h) * (dqk / 2);
      const long long bo = ((long long)h * R + rank_i) * dqk;
      qr = rotated<MIMO>(p.q + row * dqk, p.qb + bo, p.cos + cso, p.sin + cso, n0, dqk);
      kr = rotated<MIMO>(p.k + row * dqk, p.kb + bo, p.cos + cso, p.sin + cso, n0, dqk);
    }
    // ---- B-operand rows s = 4*lj + m: x (= psi v) and the update weight w
    float xv[4], wv[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const int s = 4 * lj + m;
      const int step_s = s / R;
      const long long g_s = (long long)ch * T + step_s;
      float x = 0.0f, w = 0.0f;
      if (g_s < L) {
        const long long t_s = REV ? L - 1 - g_s : g_s;
        x = p.v[(((long long)bi * L + t_s) * H + h) * dv + pcol] * psi_m[m];
        w = p.g.w[gate_base + (long long)ch * T + step_s];
      }
      xv[m] = x;
      wv[m] = w;
    }
    // ---- partial G^T = K Q^T and partial diag(e^c) Q S0^T over this wave's columns
    f4 gp = {0.0f, 0.0f, 0.0f, 0.0f}, yp = gp;
    const float ei = gi[1];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      gp = mfma(kr[r], qr[r], gp);
      yp = mfma(ei * qr[r], S[r], yp);
    }
    float* pb = part_buf + ((ch & 1) * W + wave) * 64 * 8 + lane * 8;
    *reinterpret_cast<f4*>(pb) = gp;
    *reinterpret_cast<f4*>(pb + 4) = yp;
    // ---- K transpose through LDS, then S = e^{c_last} S + K^T diag(w) X
    *reinterpret_cast<f4*>(kt + li * kKtStride + 4 * lj) = kr;
    const float etot = p.g.etot[(long long)seq * p.nchunks + ch];
    f4 acc = S * etot;
#pragma unroll
    for (int m = 0; m < 4; ++m) acc = mfma(kt[(4 * lj + m) * kKtStride + li], wv[m] * xv[m], acc);
    S = acc;
    __syncthreads();
    if (wave == 0) {
      // ---- reduce the partials, mask G, add the intra-chunk term, epilogue
      f4 G = {0.0f, 0.0f, 0.0f, 0.0f}, Y = G;
      for (int w2 = 0; w2 < W; ++w2) {
        const float* q2 = part_buf + ((ch & 1) * W + w2) * 64 * 8 + lane * 8;
        G += *reinterpret_cast<const f4*>(q2);
        Y += *reinterpret_cast<const f4*>(q2 + 4);
      }
      // lane holds G[i = li][s = 4*lj + r]
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int s = 4 * lj + r;
        const int step_s = s / R;
        const f4 gs = p.g.step[gate_base + (long long)ch * T + step_s];
        float mval = 0.0f;
        if (step_s < step_i) mval = fexp(gi[0] - gs[0]) * gs[3];
        else if (step_s == step_i) mval = gi[2];
        G[r] *= mval;
      }
#pragma unroll
      for (int m = 0; m < 4; ++m) Y = mfma(G[m], xv[m], Y);
      // lane holds Y[row = 4*lj + r][pcol]; add D x, gate, reduce ranks, store
      float o[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) o[r] = Y[r] + dskip * xv[r];
#pragma unroll
      for (int r = 0; r < 4; r += R) {
        const int s = 4 * lj + r;
        const long long g_s = (long long)ch * T + s / R;
        if (g_s < L) {
          const long long t_s = REV ? L - 1 - g_s : g_s;
          const long long vo = (((long long)bi * L + t_s) * H + h) * dv + pcol;
          const float zz = p.z ? p.z[vo] : 0.0f;
          float acc_o = 0.0f;
#pragma unroll
          for (int rr = 0; rr < R; ++rr) {
            float term = o[r + rr];
            if (p.z) term *= silu_fast(zz * zeta_r[r + rr]);
            acc_o = fmaf(phi_r[r + rr], term, acc_o);
          }
          p.out[(((long long)bi * H + h) * L + t_s) * dv + pcol] = acc_o;
        }
      }
    }
    if (ch + 1 == p.nchunks) {
      if (p.last_state)
        *reinterpret_cast<f4*>(p.last_state + ((long long)seq * dv + pcol) * dqk + n0) = S;
      if (p.last_bx && part == 0) {
        const long long gl = L - 1;  // the traversal's final step
        if (ch * (long long)T + step_i == gl && lj < 4)
          *reinterpret_cast<f4*>(p.last_bx + (long long)seq * dqk + n0) = kr * gi[3];
      }
    }
  }
}

template <int R, bool MIMO>
hipError_t launch_chunk(const M3K& k, bool rev, hipStream_t st) {
  const int W = k.dqk / 16;
  const long long blocks = 8LL * k.nparts * ((k.nseq + 7) / 8);
  const size_t lds = sizeof(float) * ((size_t)2 * W * 64 * 8 + (size_t)W * 16 * kKtStride);
  if (rev)
    hipLaunchKernelGGL((m3_chunk_kernel<R, MIMO, true>), dim3((unsigned)blocks), dim3(64 * W),
                       lds, st, k);
  else
    hipLaunchKernelGGL((m3_chunk_kernel<R, MIMO, false>), dim3((unsigned)blocks), dim3(64 * W),
                       lds, st, k);
  return hipGetLastError();
}

}  // namespace

bool m3_chunk_supported(const M3Problem& pr) {
  const bool mimo = pr.psi != nullptr;
  const bool rank_ok = mimo ? (pr.rank == 1 || pr.rank == 2 || pr.rank == 4) : pr.rank == 1;
  return rank_ok && pr.dv % 16 == 0 && pr.dqk % 16 == 0 && pr.dqk <= 256 && pr.dqk >= 16 &&
         pr.len > 0;
}

hipError_t m3_scan_chunked(const M3Problem& pr, hipStream_t st) {
  M3K k{};
  k.q = pr.q; k.k = pr.k; k.v = pr.v; k.adt = pr.adt; k.dt = pr.dt; k.trap = pr.trap;
  k.qb = pr.q_bias; k.kb = pr.k_bias; k.cos = pr.cos; k.sin = pr.sin; k.D = pr.D; k.z = pr.z;
  k.psi = pr.psi; k.zeta = pr.zeta; k.phi = pr.phi;
  k.out = pr.out; k.last_state = pr.last_state; k.last_bx = pr.last_bx;
  k.batch = (int)pr.batch; k.heads = (int)pr.heads; k.dv = (int)pr.dv; k.dqk = (int)pr.dqk;
  k.len = (int)pr.len; k.rank = (int)pr.rank; k.groups = (int)pr.groups;
  k.nparts = k.dv / 16;
  k.steps_per_chunk = 16 / k.rank;
  k.nchunks = (k.len + k.steps_per_chunk - 1) / k.steps_per_chunk;
  k.nseq = k.batch * k.heads;
  const size_t nsteps = (size_t)k.nseq * k.nchunks * k.steps_per_chunk;
  const size_t bytes = nsteps * (sizeof(f4) + sizeof(float)) + (size_t)k.nseq * k.nchunks * 4;
  char* scratch = nullptr;
  hipError_t e = hipMallocAsync((void**)&scratch, bytes, st);
  if (e != hipSuccess) return e;
  k.g.step = reinterpret_cast<f4*>(scratch);
  k.g.w = reinterpret_cast<float*>(scratch + nsteps * sizeof(f4));
  k.g.etot = k.g.w + nsteps;
  const long long gthreads = (long long)k.nseq * k.nchunks;
  hipLaunchKernelGGL(m3_gates_kernel, dim3((unsigned)((gthreads + 255) / 256)), dim3(256), 0, st,
                     k, pr.reverse ? 1 : 0);
  e = hipGetLastError();
  if (e == hipSuccess) {
    const bool rev = pr.reverse != 0;
    const bool mimo = pr.psi != nullptr;
    if (!mimo) e = launch_chunk<1, false>(k, rev, st);
    else if (k.rank == 1) e = launch_chunk<1, true>(k, rev, st);
    else if (k.rank == 2) e = launch_chunk<2, true>(k, rev, st);
    else e = launch_chunk<4, true>(k, rev, st);
  }
  const hipError_t fe = hipFreeAsync(scratch, st);
  return e != hipSuccess ? e : fe;
}

}  // namespace armscan
