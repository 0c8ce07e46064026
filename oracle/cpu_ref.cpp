// TEST INFRASTRUCTURE — NOT PART OF THE PRODUCT.
//
// CPU restatement of the reference's x86 selective-scan path
// (AdityaP9116/ARMHackathon, Rust crate `arm-scan-core` + `arm-scan-ffi`),
// written from the reference's source as text. The Rust crate cannot be built
// in this environment (no cargo/rustc, no crates.io), so this file restates
// the algorithm, the accumulation order and the libm calls it makes on x86:
//
//   Mamba-1            scalar::scan             kernel/arm-scan-core/src/scalar.rs:11-89
//   Mamba-1 bidir      scalar::scan_bidirectional  scalar.rs:114-201
//   Mamba-3 SISO       mamba3::scalar::scan     src/mamba3/scalar.rs:50-196  (naive oracle)
//                      mamba3::tiled::scan      src/mamba3/tiled.rs:278-402  (x86 Auto path)
//   Mamba-3 MIMO       mamba3::mimo::scan       src/mamba3/mimo.rs:98-284
//   numerics           Float::{softplus,silu,sigmoid}  src/float.rs:31-59
//   threading          parallel::should_parallelize*   src/parallel.rs:16-20, :91-93
//   validation / ABI   lib.rs:181-249, :304-454; mamba3/mod.rs:213-429;
//                      arm-scan-ffi/src/lib.rs:37-577
//
// Only the tests (tests/), `__graft_entry__.smoke()` and the `cpu_baseline`
// leg of bench.py load this library, always as the checker / reported CPU
// baseline and never as the thing measured or shipped.
//
// Exports
//   * the four reference C-ABI symbols with the reference's v7 host-pointer
//     signatures and return codes (`arm_scan_*_f32`, ABI 7);
//   * f64 twins of the same entry points (`arm_scan_*_f64`), used to pin this
//     restatement against the reference's float64 golden vectors;
//   * `oracle_mamba3_scan_{f32,f64}`: the Mamba-3 entry point widened with the
//     two extensions the MI355X library adds (a q/k `groups` axis and a MIMO
//     final state), so the GPU path can be checked at the benchmark shapes.
//
// Arithmetic follows the reference exactly: no FMA contraction (the build
// passes -ffp-contract=off and targets baseline x86-64, which has no FMA),
// glibc expf/log1pf (Rust's f32::exp / f32::ln_1p on x86 Linux call them), and
// the same per-element operation order as the Rust loops.

#include <cmath>
#include <cstddef>
#include <cstdint>
#include <algorithm>
#include <cstring>
#include <thread>
#include <tuple>
#include <vector>

namespace {

// ---------------------------------------------------------------- numerics
// float.rs:31-59. `Float::exp` / `Float::ln_1p` are the platform libm calls.
template <class T> struct M;
template <> struct M<float> {
  static float exp(float x) { return expf(x); }
  static float ln_1p(float x) { return log1pf(x); }
};
template <> struct M<double> {
  static double exp(double x) { return ::exp(x); }
  static double ln_1p(double x) { return ::log1p(x); }
};

template <class T> inline T softplus(T x) {  // float.rs:31-37, threshold 20 (:85)
  return x > T(20) ? x : M<T>::ln_1p(M<T>::exp(x));
}
template <class T> inline T silu(T x) {  // float.rs:41-43
  return x / (T(1) + M<T>::exp(-x));
}
template <class T> inline T sigmoid(T x) {  // float.rs:52-59
  if (x >= T(0)) return T(1) / (T(1) + M<T>::exp(-x));
  T e = M<T>::exp(x);
  return e / (T(1) + e);
}

// ---------------------------------------------------------------- threading
// parallel.rs:16-20 and :91-93. Rows are independent, so the result is
// bit-identical whatever the thread count (property.rs:453-497).
constexpr size_t kParallelWorkThreshold = size_t(1) << 17;

enum Threading { TH_AUTO = 0, TH_SEQ = 1, TH_RAYON = 2 };

// Worker count for the parallel path (Rayon's default is one per logical CPU).
int g_threads = 0;
int worker_count() {
  if (g_threads > 0) return g_threads;
  unsigned n = std::thread::hardware_concurrency();
  return n ? (int)n : 1;
}

// Static partition of [0, n) over the workers, each with its own scratch —
// the same row-disjoint decomposition as parallel::for_each_channel
// (parallel.rs:24-85). `Body(scratch, row)`; `Init()` builds the scratch.
template <class Init, class Body>
void for_rows(bool par, size_t n, Init init, Body body) {
  const int workers = par ? (int)std::min<size_t>((size_t)worker_count(), n) : 1;
  if (workers <= 1) {
    auto s = init();
    for (size_t i = 0; i < n; ++i) body(s, i);
    return;
  }
  std::vector<std::thread> pool;
  pool.reserve(workers);
  for (int w = 0; w < workers; ++w) {
    const size_t lo = n * (size_t)w / (size_t)workers, hi = n * (size_t)(w + 1) / (size_t)workers;
    pool.emplace_back([&, lo, hi]() {
      auto s = init();
      for (size_t i = lo; i < hi; ++i) body(s, i);
    });
  }
  for (auto& t : pool) t.join();
}

bool par_channels(int threading, size_t n_channels, size_t len, size_t state) {
  if (threading == TH_SEQ) return false;
  if (threading == TH_RAYON) return true;
  return n_channels >= 2 && n_channels * len * state >= kParallelWorkThreshold;
}
bool par_heads(int threading, size_t n_heads, size_t len, size_t dv, size_t dqk) {
  if (threading == TH_SEQ) return false;
  if (threading == TH_RAYON) return true;
  // saturating product as in parallel.rs:92
  long double w = (long double)n_heads * (long double)len * (long double)(dv * dqk);
  return n_heads >= 2 && w >= (long double)kParallelWorkThreshold;
}

// ---------------------------------------------------------------- ABI types
// arm-scan-ffi/src/lib.rs:43-58, :362-373
struct ArmScanDims {
  size_t batch, dim, len, state, groups;
};
struct ArmMamba3Dims {
  size_t batch, heads, dv, dqk, len, rank;
};

enum Code {
  OK = 0,
  ERR_NULL = 1,
  ERR_DIMS = 2,
  ERR_BACKEND = 3,
  ERR_ENUM = 4,
};

bool mul_ok(size_t a, size_t b, size_t* out) {
  return !__builtin_mul_overflow(a, b, out);
}
bool mul3(size_t a, size_t b, size_t c, size_t* out) {
  size_t t;
  return mul_ok(a, b, &t) && mul_ok(t, c, out);
}
bool mul4(size_t a, size_t b, size_t c, size_t d, size_t* out) {
  size_t t;
  return mul3(a, b, c, &t) && mul_ok(t, d, out);
}

// backend: 0 auto, 1 scalar, 2 neon (arm-scan-ffi/src/lib.rs:60-67)
bool backend_ok(int b) { return b >= 0 && b <= 2; }
bool threading_ok(int t) { return t >= 0 && t <= 2; }

// ---------------------------------------------------------------- Mamba-1
template <class T> struct M1In {
  const T *u, *delta, *a, *b, *c, *d_skip, *z, *delta_bias;
  bool softplus_on, reverse;
};

// scalar.rs:11-89 — one (batch, channel) row per iteration.
template <class T>
void m1_scan(const ArmScanDims& d, const M1In<T>& in, const T* h0, T* out, T* last,
             int threading) {
  const size_t dim = d.dim, len = d.len, state = d.state, groups = d.groups;
  const size_t group_size = dim / groups;
  const size_t n_ch = d.batch * dim;
  const bool par = par_channels(threading, n_ch, len, state);
  for_rows(par, n_ch, [&] { return std::make_tuple(std::vector<T>(state)); },
           [&](auto& sc, size_t ch) {
      auto& [h] = sc;
      const size_t bi = ch / dim, dd = ch % dim;
      const T* a_row = in.a + dd * state;
      const T bias = in.delta_bias ? in.delta_bias[dd] : T(0);
      const size_t bc_base = (bi * groups + dd / group_size) * state * len;
      const size_t row = ch * len;
      const T* u_row = in.u + row;
      const T* dl_row = in.delta + row;
      const T* z_row = in.z ? in.z + row : nullptr;
      T* o_row = out + row;
      if (h0)
        for (size_t n = 0; n < state; ++n) h[n] = h0[ch * state + n];
      else
        for (size_t n = 0; n < state; ++n) h[n] = T(0);
      for (size_t i = 0; i < len; ++i) {
        const size_t t = in.reverse ? len - 1 - i : i;
        T dt = dl_row[t] + bias;
        if (in.softplus_on) dt = softplus(dt);
        const T dt_u = dt * u_row[t];
        T y = T(0);
        for (size_t n = 0; n < state; ++n) {
          const size_t bc = bc_base + n * len + t;
          const T nw = M<T>::exp(dt * a_row[n]) * h[n] + dt_u * in.b[bc];
          h[n] = nw;
          y = y + in.c[bc] * nw;
        }
        if (in.d_skip) y = y + in.d_skip[dd] * u_row[t];
        if (z_row) y = y * silu(z_row[t]);
        o_row[t] = y;
      }
      if (last)
        for (size_t n = 0; n < state; ++n) last[ch * state + n] = h[n];
  });
}

// scalar.rs:114-201 — Pass A (abar, bbar) once per row, then both directions.
template <class T>
void m1_scan_bidir(const ArmScanDims& d, const M1In<T>& in, T* out_f, T* out_b, T* last_f,
                   T* last_b, int threading) {
  const size_t dim = d.dim, len = d.len, state = d.state, groups = d.groups;
  const size_t group_size = dim / groups;
  const size_t n_ch = d.batch * dim;
  const bool par = par_channels(threading, n_ch, len, state);
  for_rows(par, n_ch, [&] { return std::make_tuple(std::vector<T>(len * state), std::vector<T>(len * state), std::vector<T>(state)); },
           [&](auto& sc, size_t ch) {
      auto& [abar, bbar, h] = sc;
      const size_t bi = ch / dim, dd = ch % dim;
      const T* a_row = in.a + dd * state;
      const T bias = in.delta_bias ? in.delta_bias[dd] : T(0);
      const size_t bc_base = (bi * groups + dd / group_size) * state * len;
      const size_t row = ch * len;
      const T* u_row = in.u + row;
      const T* dl_row = in.delta + row;
      const T* z_row = in.z ? in.z + row : nullptr;
      for (size_t t = 0; t < len; ++t) {
        T dt = dl_row[t] + bias;
        if (in.softplus_on) dt = softplus(dt);
        const T dt_u = dt * u_row[t];
        for (size_t n = 0; n < state; ++n) {
          const size_t bc = bc_base + n * len + t;
          abar[t * state + n] = M<T>::exp(dt * a_row[n]);
          bbar[t * state + n] = dt_u * in.b[bc];
        }
      }
      for (int dir = 0; dir < 2; ++dir) {
        const bool rev = dir == 1;
        T* o_row = (rev ? out_b : out_f) + row;
        T* last = rev ? last_b : last_f;
        for (size_t n = 0; n < state; ++n) h[n] = T(0);
        for (size_t i = 0; i < len; ++i) {
          const size_t t = rev ? len - 1 - i : i;
          T y = T(0);
          for (size_t n = 0; n < state; ++n) {
            const T nw = abar[t * state + n] * h[n] + bbar[t * state + n];
            h[n] = nw;
            y = y + in.c[bc_base + n * len + t] * nw;
          }
          if (in.d_skip) y = y + in.d_skip[dd] * u_row[t];
          if (z_row) y = y * silu(z_row[t]);
          o_row[t] = y;
        }
        if (last)
          for (size_t n = 0; n < state; ++n) last[ch * state + n] = h[n];
      }
  });
}

template <class T>
int m1_entry(const ArmScanDims* dims, const T* u, const T* delta, const T* a, const T* b,
             const T* c, const T* d_skip, const T* z, const T* delta_bias, int delta_softplus,
             int reverse, int backend, int threading, T* out, T* last_state, const T* h0) {
  // arm-scan-ffi/src/lib.rs:117-158
  if (!dims || !u || !delta || !a || !b || !c || !out) return ERR_NULL;
  if (!backend_ok(backend) || !threading_ok(threading)) return ERR_ENUM;
  const ArmScanDims& d = *dims;
  size_t tmp;
  if (!mul3(d.batch, d.dim, d.len, &tmp) || !mul4(d.batch, d.groups, d.state, d.len, &tmp) ||
      !mul_ok(d.dim, d.state, &tmp) || !mul3(d.batch, d.dim, d.state, &tmp))
    return ERR_DIMS;
  // lib.rs:181-207 (lengths are exact by construction at the FFI)
  if (!d.batch || !d.dim || !d.len || !d.state || !d.groups) return ERR_DIMS;
  if (d.dim % d.groups) return ERR_DIMS;
  // lib.rs:325-345: Neon is aarch64-only; Auto resolves to scalar on x86.
  if (backend == 2) return ERR_BACKEND;
  M1In<T> in{u, delta, a, b, c, d_skip, z, delta_bias, delta_softplus != 0, reverse != 0};
  m1_scan<T>(d, in, h0, out, last_state, threading);
  return OK;
}

template <class T>
int m1_bidir_entry(const ArmScanDims* dims, const T* u, const T* delta, const T* a,
                   const T* b, const T* c, const T* d_skip, const T* z, const T* delta_bias,
                   int delta_softplus, int backend, int threading, T* out_fwd, T* out_bwd,
                   T* last_fwd, T* last_bwd) {
  // arm-scan-ffi/src/lib.rs:253-354, lib.rs:363-454
  if (!dims || !u || !delta || !a || !b || !c || !out_fwd || !out_bwd) return ERR_NULL;
  if (!backend_ok(backend) || !threading_ok(threading)) return ERR_ENUM;
  const ArmScanDims& d = *dims;
  size_t tmp;
  if (!mul3(d.batch, d.dim, d.len, &tmp) || !mul4(d.batch, d.groups, d.state, d.len, &tmp) ||
      !mul_ok(d.dim, d.state, &tmp) || !mul3(d.batch, d.dim, d.state, &tmp))
    return ERR_DIMS;
  if (!d.batch || !d.dim || !d.len || !d.state || !d.groups) return ERR_DIMS;
  if (d.dim % d.groups) return ERR_DIMS;
  // last_fwd / last_bwd both or neither -> a shape error (lib.rs:391-399)
  if ((last_fwd != nullptr) != (last_bwd != nullptr)) return ERR_DIMS;
  if (backend == 2) return ERR_BACKEND;
  M1In<T> in{u, delta, a, b, c, d_skip, z, delta_bias, delta_softplus != 0, false};
  m1_scan_bidir<T>(d, in, out_fwd, out_bwd, last_fwd, last_bwd, threading);
  return OK;
}

// ---------------------------------------------------------------- Mamba-3
template <class T> struct M3In {
  const T *q, *k, *v, *adt, *dt, *trap, *q_bias, *k_bias, *cos, *sin, *d_skip, *z;
  const T *psi, *zeta, *phi;  // all null (SISO) or all set (MIMO)
  bool reverse;
};

struct M3Shape {
  size_t batch, heads, dv, dqk, len, rank, groups;
};

// q/k element offset of (bi, t, r, group of head h, 0). The reference layout
// is (b, l, rank, 1, dqk) (mamba3/mod.rs:47-57, mimo.rs:162-163); the MI355X
// extension adds a groups axis after rank: (b, l, rank, groups, dqk), head h
// reading group h / (heads / groups). groups == 1 is the reference layout.
inline size_t qk_off(const M3Shape& s, size_t bi, size_t t, size_t r, size_t h) {
  const size_t g = h / (s.heads / s.groups);
  return (((bi * s.len + t) * s.rank + r) * s.groups + g) * s.dqk;
}

// The trapezoid gate shared by all three Mamba-3 kernels:
// mamba3/scalar.rs:95-115 (tiled.rs:317-331, mimo.rs:142-155 are identical).
template <class T>
inline void m3_gates(const M3In<T>& in, size_t gate_base, size_t len, size_t i, size_t t,
                     T* gamma, T* scale, T* alpha) {
  const size_t g = gate_base + t;
  const T lam = sigmoid(in.trap[g]);
  *gamma = in.dt[g] * lam;
  bool has_nxt;
  size_t nxt = 0;
  if (in.reverse) {
    has_nxt = i + 1 < len;
    if (has_nxt) nxt = gate_base + t - 1;
  } else {
    has_nxt = t + 1 < len;
    if (has_nxt) nxt = g + 1;
  }
  const T shifted = has_nxt ? in.dt[nxt] * (T(1) - sigmoid(in.trap[nxt])) : T(0);
  *scale = *gamma + shifted;
  *alpha = M<T>::exp(in.adt[g]);
}

// Interleaved RoPE, pairs (2i, 2i+1): mamba3/scalar.rs:40-48, tiled.rs:268-276.
template <class T>
inline void rope_interleaved(const T* src, const T* bias, const T* cs, const T* sn, T* dst,
                             size_t dqk) {
  for (size_t i = 0; i < dqk / 2; ++i) {
    const T a = src[2 * i] + bias[2 * i], b = src[2 * i + 1] + bias[2 * i + 1];
    const T c = cs[i], s = sn[i];
    dst[2 * i] = a * c - b * s;
    dst[2 * i + 1] = a * s + b * c;
  }
}

// Split-halves RoPE, pairs (i, i + dqk/2) for i < len(cos): mimo.rs:83-96.
template <class T>
inline void rope_split_halves(const T* src, const T* bias, const T* cs, const T* sn, T* dst,
                              size_t dqk, size_t n_angles) {
  const size_t half = dqk / 2;
  const size_t pairs = n_angles < half ? n_angles : half;
  for (size_t i = 0; i < dqk; ++i) dst[i] = src[i] + bias[i];
  for (size_t i = 0; i < pairs; ++i) {
    const T a = dst[i], b = dst[half + i];
    const T c = cs[i], s = sn[i];
    dst[i] = a * c - b * s;
    dst[half + i] = a * s + b * c;
  }
}

// mamba3/scalar.rs:50-196 — the naive SISO oracle (Backend::Scalar).
template <class T>
void m3_siso_naive(const M3Shape& s, const M3In<T>& in, T* out, T* last_s, T* last_bx,
                   int threading) {
  const size_t heads = s.heads, dv = s.dv, dqk = s.dqk, len = s.len, half = dqk / 2;
  const size_t n_bh = s.batch * heads;
  const bool par = par_heads(threading, n_bh, len, dv, dqk);
  for_rows(par, n_bh, [&] { return std::make_tuple(std::vector<T>(dv * dqk), std::vector<T>(dqk), std::vector<T>(dqk), std::vector<T>(dqk)); },
           [&](auto& sc, size_t bh) {
      auto& [S, q, k, bx] = sc;
      const size_t bi = bh / heads, h = bh % heads;
      const T* qb = in.q_bias + h * dqk;
      const T* kb = in.k_bias + h * dqk;
      const T d_skip = in.d_skip ? in.d_skip[h] : T(0);
      const size_t gate_base = (bi * heads + h) * len;
      T* o_row = out + bh * len * dv;  // head-major (b, h, l, dv)
      std::fill(S.begin(), S.end(), T(0));
      std::fill(bx.begin(), bx.end(), T(0));
      for (size_t i = 0; i < len; ++i) {
        const size_t t = in.reverse ? len - 1 - i : i;
        T gamma, scale, alpha;
        m3_gates(in, gate_base, len, i, t, &gamma, &scale, &alpha);
        const size_t cs_off = ((bi * len + t) * heads + h) * half;
        const size_t qo = qk_off(s, bi, t, 0, h);
        rope_interleaved(in.q + qo, qb, in.cos + cs_off, in.sin + cs_off, q.data(), dqk);
        rope_interleaved(in.k + qo, kb, in.cos + cs_off, in.sin + cs_off, k.data(), dqk);
        const size_t v_off = ((bi * len + t) * heads + h) * dv;
        const T* v = in.v + v_off;
        T qk = T(0);
        for (size_t j = 0; j < dqk; ++j) qk = qk + q[j] * k[j];
        const T diag = d_skip + gamma * qk;
        T* dst = o_row + t * dv;
        for (size_t p = 0; p < dv; ++p) {
          T acc = T(0);
          for (size_t j = 0; j < dqk; ++j) acc = acc + q[j] * S[p * dqk + j];
          dst[p] = alpha * acc + diag * v[p];
        }
        for (size_t p = 0; p < dv; ++p) {
          const T sv = scale * v[p];
          for (size_t j = 0; j < dqk; ++j) S[p * dqk + j] = alpha * S[p * dqk + j] + sv * k[j];
        }
        for (size_t j = 0; j < dqk; ++j) bx[j] = scale * k[j];
        if (in.z) {
          const T* zs = in.z + v_off;
          for (size_t p = 0; p < dv; ++p) dst[p] = dst[p] * silu(zs[p]);
        }
      }
      if (last_s) std::memcpy(last_s + bh * dv * dqk, S.data(), dv * dqk * sizeof(T));
      if (last_bx) std::memcpy(last_bx + bh * dqk, bx.data(), dqk * sizeof(T));
  });
}

// mamba3/tiled.rs:278-402 — the blocked twin, x86 Backend::Auto for SISO.
template <class T>
void m3_siso_tiled(const M3Shape& s, const M3In<T>& in, T* out, T* last_s, T* last_bx,
                   int threading) {
  constexpr size_t TILE = 32;  // tiled.rs:246
  const size_t heads = s.heads, dv = s.dv, dqk = s.dqk, len = s.len, half = dqk / 2;
  const size_t n_bh = s.batch * heads;
  const bool par = par_heads(threading, n_bh, len, dv, dqk);
  for_rows(par, n_bh, [&] { return std::make_tuple(std::vector<T>(dv * dqk), std::vector<T>(dqk), std::vector<T>(dqk), std::vector<T>(dv), std::vector<T>(dqk)); },
           [&](auto& sc, size_t bh) {
      auto& [S, q, k, y, bx] = sc;
      const size_t bi = bh / heads, h = bh % heads;
      const T* qb = in.q_bias + h * dqk;
      const T* kb = in.k_bias + h * dqk;
      const T d_skip = in.d_skip ? in.d_skip[h] : T(0);
      const size_t gate_base = (bi * heads + h) * len;
      T* o_row = out + bh * len * dv;
      std::fill(S.begin(), S.end(), T(0));
      std::fill(bx.begin(), bx.end(), T(0));
      for (size_t i = 0; i < len; ++i) {
        const size_t t = in.reverse ? len - 1 - i : i;
        T gamma, scale, alpha;
        m3_gates(in, gate_base, len, i, t, &gamma, &scale, &alpha);
        const size_t cs_off = ((bi * len + t) * heads + h) * half;
        const size_t qo = qk_off(s, bi, t, 0, h);
        rope_interleaved(in.q + qo, qb, in.cos + cs_off, in.sin + cs_off, q.data(), dqk);
        rope_interleaved(in.k + qo, kb, in.cos + cs_off, in.sin + cs_off, k.data(), dqk);
        const size_t v_off = ((bi * len + t) * heads + h) * dv;
        const T* v = in.v + v_off;
        T qk = T(0);
        for (size_t j = 0; j < dqk; ++j) qk = qk + q[j] * k[j];
        const T diag = d_skip + gamma * qk;
        std::fill(y.begin(), y.end(), T(0));
        for (size_t c0 = 0; c0 < dqk; c0 += TILE) {
          const size_t c1 = c0 + TILE < dqk ? c0 + TILE : dqk;
          for (size_t r = 0; r < dv; ++r) {
            const T sv = scale * v[r];
            T acc = T(0);
            T* row = S.data() + r * dqk;
            for (size_t j = c0; j < c1; ++j) {
              const T old = row[j];
              acc = acc + q[j] * old;
              row[j] = alpha * old + sv * k[j];
            }
            y[r] = y[r] + acc;
          }
        }
        T* dst = o_row + t * dv;
        for (size_t p = 0; p < dv; ++p) dst[p] = alpha * y[p] + diag * v[p];
        for (size_t j = 0; j < dqk; ++j) bx[j] = scale * k[j];
        if (in.z) {
          const T* zs = in.z + v_off;
          for (size_t p = 0; p < dv; ++p) dst[p] = dst[p] * silu(zs[p]);
        }
      }
      if (last_s) std::memcpy(last_s + bh * dv * dqk, S.data(), dv * dqk * sizeof(T));
      if (last_bx) std::memcpy(last_bx + bh * dqk, bx.data(), dqk * sizeof(T));
  });
}

// mamba3/mimo.rs:98-284 — rank-r MIMO with one shared state per (b, h).
// `last_s` is the MI355X extension (the reference rejects a MIMO carry,
// mamba3/mod.rs:261-268); it is the state after the final traversal step,
// exactly what the SISO paths write.
template <class T>
void m3_mimo(const M3Shape& s, const M3In<T>& in, T* out, T* last_s, int threading) {
  const size_t heads = s.heads, dv = s.dv, dqk = s.dqk, len = s.len, rank = s.rank;
  const size_t half = dqk / 2;
  const size_t n_bh = s.batch * heads;
  const bool par = par_heads(threading, n_bh, len, dv, dqk);
  for_rows(par, n_bh, [&] { return std::make_tuple(std::vector<T>(dv * dqk), std::vector<T>(rank * dqk), std::vector<T>(rank * dqk), std::vector<T>(rank * dv), std::vector<T>(rank * dv), std::vector<T>(rank * rank)); },
           [&](auto& sc, size_t bh) {
      auto& [S, q, k, x, acc, qk] = sc;
      const size_t bi = bh / heads, h = bh % heads;
      const size_t bias_base = h * rank * dqk;
      const size_t proj_base = h * rank * dv;
      const T d_skip = in.d_skip ? in.d_skip[h] : T(0);
      const size_t gate_base = (bi * heads + h) * len;
      T* o_row = out + bh * len * dv;
      std::fill(S.begin(), S.end(), T(0));
      for (size_t i = 0; i < len; ++i) {
        const size_t t = in.reverse ? len - 1 - i : i;
        T gamma, scale, alpha;
        m3_gates(in, gate_base, len, i, t, &gamma, &scale, &alpha);
        const size_t cs_off = ((bi * len + t) * heads + h) * half;
        for (size_t r = 0; r < rank; ++r) {
          const size_t src = qk_off(s, bi, t, r, h);
          const size_t b0 = bias_base + r * dqk;
          rope_split_halves(in.q + src, in.q_bias + b0, in.cos + cs_off, in.sin + cs_off,
                            q.data() + r * dqk, dqk, half);
          rope_split_halves(in.k + src, in.k_bias + b0, in.cos + cs_off, in.sin + cs_off,
                            k.data() + r * dqk, dqk, half);
        }
        const size_t v_off = ((bi * len + t) * heads + h) * dv;
        const T* v = in.v + v_off;
        for (size_t r = 0; r < rank; ++r)
          for (size_t p = 0; p < dv; ++p)
            x[r * dv + p] = in.psi[proj_base + r * dv + p] * v[p];
        for (size_t a = 0; a < rank; ++a)
          for (size_t b = 0; b < rank; ++b) {
            T sum = T(0);
            for (size_t j = 0; j < dqk; ++j) sum = sum + q[a * dqk + j] * k[b * dqk + j];
            qk[a * rank + b] = sum;
          }
        for (size_t r = 0; r < rank; ++r) {
          const T* qr = q.data() + r * dqk;
          for (size_t p = 0; p < dv; ++p) {
            T a = T(0);
            for (size_t j = 0; j < dqk; ++j) a = a + qr[j] * S[p * dqk + j];
            T dsum = T(0);
            for (size_t b = 0; b < rank; ++b) dsum = dsum + qk[r * rank + b] * x[b * dv + p];
            acc[r * dv + p] = alpha * a + gamma * dsum + d_skip * x[r * dv + p];
          }
        }
        for (size_t p = 0; p < dv; ++p)
          for (size_t n = 0; n < dqk; ++n) {
            T upd = T(0);
            for (size_t r = 0; r < rank; ++r) upd = upd + x[r * dv + p] * k[r * dqk + n];
            S[p * dqk + n] = alpha * S[p * dqk + n] + scale * upd;
          }
        T* dst = o_row + t * dv;
        for (size_t p = 0; p < dv; ++p) dst[p] = T(0);
        for (size_t r = 0; r < rank; ++r) {
          const T* phi = in.phi + proj_base + r * dv;
          const T* zeta = in.zeta + proj_base + r * dv;
          const T* ar = acc.data() + r * dv;
          if (in.z) {
            const T* zs = in.z + v_off;
            for (size_t p = 0; p < dv; ++p) dst[p] = dst[p] + phi[p] * silu(zs[p] * zeta[p]) * ar[p];
          } else {
            for (size_t p = 0; p < dv; ++p) dst[p] = dst[p] + phi[p] * ar[p];
          }
        }
      }
      if (last_s) std::memcpy(last_s + bh * dv * dqk, S.data(), dv * dqk * sizeof(T));
  });
}

// Shared validation + routing for the v7 entry point and its widened twin.
// `extended` enables the MI355X-only extensions (groups > 1, MIMO last_state).
template <class T>
int m3_entry(const M3Shape& s, const M3In<T>& in, int backend, int threading, T* out,
             T* last_state, T* last_bx, bool extended) {
  if (!in.q || !in.k || !in.v || !in.adt || !in.dt || !in.trap || !in.q_bias || !in.k_bias ||
      !in.cos || !in.sin || !out)
    return ERR_NULL;
  const int n_mimo = (in.psi != nullptr) + (in.zeta != nullptr) + (in.phi != nullptr);
  const bool mimo = n_mimo == 3;
  // arm-scan-ffi/src/lib.rs:462-473: half a carry / partial projections -> 1.
  // The widened entry allows a MIMO last_state without last_bx.
  if (!(extended && mimo) && (last_state == nullptr) != (last_bx == nullptr)) return ERR_NULL;
  if (n_mimo != 0 && n_mimo != 3) return ERR_NULL;
  if (!backend_ok(backend) || !threading_ok(threading)) return ERR_ENUM;
  if (s.dqk % 2) return ERR_DIMS;
  if (s.rank == 0) return ERR_DIMS;
  size_t tmp;
  if (!mul4(s.batch, s.len, s.rank, s.dqk, &tmp) || !mul_ok(tmp, s.groups, &tmp) ||
      !mul3(s.batch, s.heads, s.len, &tmp) || !mul3(s.heads, s.rank, s.dqk, &tmp) ||
      !mul3(s.heads, s.rank, s.dv, &tmp) || !mul4(s.batch, s.len, s.heads, s.dv, &tmp) ||
      !mul4(s.batch, s.heads, s.dv, s.dqk, &tmp))
    return ERR_DIMS;
  // mamba3/mod.rs:228-276
  if (!s.batch || !s.heads || !s.dv || !s.dqk || !s.len || !s.rank || !s.groups) return ERR_DIMS;
  if (s.heads % s.groups) return ERR_DIMS;
  if (s.rank > 1 && !mimo) return ERR_DIMS;
  if (mimo && last_bx) return ERR_DIMS;
  if (mimo && last_state && !extended) return ERR_DIMS;
  // mamba3/mod.rs:383-386: MIMO always goes to mimo::scan, before the
  // backend match; SISO Scalar -> naive, Auto -> tiled (x86), Neon -> 3.
  if (mimo) {
    m3_mimo<T>(s, in, out, last_state, threading);
    return OK;
  }
  if (backend == 2) return ERR_BACKEND;
  if (backend == 1)
    m3_siso_naive<T>(s, in, out, last_state, last_bx, threading);
  else
    m3_siso_tiled<T>(s, in, out, last_state, last_bx, threading);
  return OK;
}

template <class T>
int m3_v7_entry(const ArmMamba3Dims* dims, const T* q, const T* k, const T* v, const T* adt,
                const T* dt, const T* trap, const T* q_bias, const T* k_bias, const T* cos,
                const T* sin, const T* d_skip, const T* z, const T* psi, const T* zeta,
                const T* phi, int reverse, int backend, int threading, T* out, T* last_state,
                T* last_bx) {
  if (!dims) return ERR_NULL;
  const M3Shape s{dims->batch, dims->heads, dims->dv, dims->dqk, dims->len, dims->rank, 1};
  const M3In<T> in{q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z,
                   psi, zeta, phi, reverse != 0};
  return m3_entry<T>(s, in, backend, threading, out, last_state, last_bx, false);
}

}  // namespace

extern "C" {

// Dims of the widened Mamba-3 entry point: the v7 struct plus `groups`.
struct OracleMamba3Dims {
  size_t batch, heads, dv, dqk, len, rank, groups;
};

uint32_t arm_scan_abi_version(void) { return 7; }

int arm_scan_selective_scan_f32(const ArmScanDims* dims, const float* u, const float* delta,
                                const float* a, const float* b, const float* c,
                                const float* d_skip, const float* z, const float* delta_bias,
                                int delta_softplus, int reverse, int backend, int threading,
                                float* out, float* last_state, const float* h0) {
  return m1_entry<float>(dims, u, delta, a, b, c, d_skip, z, delta_bias, delta_softplus,
                         reverse, backend, threading, out, last_state, h0);
}
int arm_scan_selective_scan_f64(const ArmScanDims* dims, const double* u, const double* delta,
                                const double* a, const double* b, const double* c,
                                const double* d_skip, const double* z, const double* delta_bias,
                                int delta_softplus, int reverse, int backend, int threading,
                                double* out, double* last_state, const double* h0) {
  return m1_entry<double>(dims, u, delta, a, b, c, d_skip, z, delta_bias, delta_softplus,
                          reverse, backend, threading, out, last_state, h0);
}

int arm_scan_selective_scan_bidirectional_f32(
    const ArmScanDims* dims, const float* u, const float* delta, const float* a,
    const float* b, const float* c, const float* d_skip, const float* z,
    const float* delta_bias, int delta_softplus, int backend, int threading, float* out_fwd,
    float* out_bwd, float* last_fwd, float* last_bwd) {
  return m1_bidir_entry<float>(dims, u, delta, a, b, c, d_skip, z, delta_bias, delta_softplus,
                               backend, threading, out_fwd, out_bwd, last_fwd, last_bwd);
}
int arm_scan_selective_scan_bidirectional_f64(
    const ArmScanDims* dims, const double* u, const double* delta, const double* a,
    const double* b, const double* c, const double* d_skip, const double* z,
    const double* delta_bias, int delta_softplus, int backend, int threading, double* out_fwd,
    double* out_bwd, double* last_fwd, double* last_bwd) {
  return m1_bidir_entry<double>(dims, u, delta, a, b, c, d_skip, z, delta_bias,
                                delta_softplus, backend, threading, out_fwd, out_bwd, last_fwd,
                                last_bwd);
}

int arm_scan_mamba3_scan_f32(const ArmMamba3Dims* dims, const float* q, const float* k,
                             const float* v, const float* adt, const float* dt,
                             const float* trap, const float* q_bias, const float* k_bias,
                             const float* cos, const float* sin, const float* d_skip,
                             const float* z, const float* psi, const float* zeta,
                             const float* phi, int reverse, int backend, int threading,
                             float* out, float* last_state, float* last_bx) {
  return m3_v7_entry<float>(dims, q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z,
                            psi, zeta, phi, reverse, backend, threading, out, last_state,
                            last_bx);
}
int arm_scan_mamba3_scan_f64(const ArmMamba3Dims* dims, const double* q, const double* k,
                             const double* v, const double* adt, const double* dt,
                             const double* trap, const double* q_bias, const double* k_bias,
                             const double* cos, const double* sin, const double* d_skip,
                             const double* z, const double* psi, const double* zeta,
                             const double* phi, int reverse, int backend, int threading,
                             double* out, double* last_state, double* last_bx) {
  return m3_v7_entry<double>(dims, q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip,
                             z, psi, zeta, phi, reverse, backend, threading, out, last_state,
                             last_bx);
}

#define ORACLE_M3_EXT(T, NAME)                                                               \
  int NAME(const OracleMamba3Dims* dims, const T* q, const T* k, const T* v, const T* adt,   \
           const T* dt, const T* trap, const T* q_bias, const T* k_bias, const T* cos,       \
           const T* sin, const T* d_skip, const T* z, const T* psi, const T* zeta,           \
           const T* phi, int reverse, int backend, int threading, T* out, T* last_state,     \
           T* last_bx) {                                                                     \
    if (!dims) return ERR_NULL;                                                              \
    const M3Shape s{dims->batch, dims->heads, dims->dv,   dims->dqk,                         \
                    dims->len,   dims->rank,  dims->groups};                                 \
    const M3In<T> in{q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z,            \
                     psi, zeta, phi, reverse != 0};                                          \
    return m3_entry<T>(s, in, backend, threading, out, last_state, last_bx, true);           \
  }
ORACLE_M3_EXT(float, oracle_mamba3_scan_f32)
ORACLE_M3_EXT(double, oracle_mamba3_scan_f64)

int oracle_set_threads(int n) {
  if (n > 0) g_threads = n;
  return worker_count();
}

}  // extern "C"
