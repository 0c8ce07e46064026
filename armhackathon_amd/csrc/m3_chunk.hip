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
// Two kernels:
//  * m3_gates_kernel, one lane per (sequence, chunk, row): the chunk's gate record
//    {M, e^c, w, e^{c_last}} (1168 bytes per chunk at rank 1, 112 at rank 4), so that
//    the main kernel does no transcendental work for the decays.
//  * m3_chunk_kernel: one block per (sequence, PT 16-column slices of dv), one
//    wave per 16-column slice of dqk (an "n-tile"). A wave keeps the PT 16x16
//    pieces S[slice][n-tile] in MFMA registers and per chunk computes
//      its partial G^T = K Q^T over its n-tile (4 MFMA),
//      per slice its partial Q S0^T (4 MFMA),
//      per slice the update of its S piece (4 MFMA, K transposed through LDS).
//    The partials meet in LDS; two epilogue waves per slice, one for the even
//    chunks and one for the odd, finish a chunk over the next two chunks' time:
//    the reduction of the partials, then the masked intra-chunk term (4 MFMA), D x,
//    gating, rank sum, store.
//
// Every input of a chunk (q, k, cos, sin, v and z rows and the gate record)
// reaches LDS by direct-to-LDS DMA (global_load_lds_dwordx4) NS-1 chunks ahead,
// through a ring of NS stages (as many as fit in LDS, at most kStages): no VGPRs
// are spent on staging and HBM latency stays off the chunk loop. Each wave waits with an explicit vmcnt for its own
// share of a stage, and a workgroup barrier publishes the stage. Rows of the last
// chunk past the end of the sequence are clamped to the last step on load (their
// gates are zero, so they add nothing) and are not stored.
//
// Every MFMA operand is used in the register layout the previous MFMA produced:
// the reduction index of each product is permuted so that lane l (row l%16,
// group j = l/16) always supplies element (l%16, 4j + r).

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <type_traits>

#include "scan_common.h"
#include "scan_launch.h"

namespace armscan {

namespace {

typedef float f4 __attribute__((ext_vector_type(4)));
typedef float f2 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ f4 mfma(float a, float b, f4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Gate record of one (sequence, chunk) of T = 16/R steps, in floats. The rows of a
// step share its gates, so M is kept over step pairs, e^{c} and w per step:
//   M[step_i][step_s] (T x T), e^{c} (T), w (T), e^{c_last}, padding to whole
//   16-byte pieces; with the angle pre-pass fused, dt / 2 of each of the 16 rows
//   (the rotation per unit of tanh(angle), pi * dt radians, in turns).
// Rank 1: 292 floats (1168 bytes), rank 2: 84, rank 4: 28 (112 bytes).
template <int R> struct Rec {
  static constexpr int T = 16 / R;
  static constexpr int M = 0, Ec = T * T, W = Ec + T, Etot = W + T;
  static constexpr int Floats = (Etot + 1 + 3) & ~3;
  static constexpr int Hdt = Floats, FloatsAng = Floats + 16;
};
constexpr int rec_floats(int R, bool ang) {
  return R == 1 ? (ang ? Rec<1>::FloatsAng : Rec<1>::Floats)
                : R == 2 ? (ang ? Rec<2>::FloatsAng : Rec<2>::Floats)
                         : (ang ? Rec<4>::FloatsAng : Rec<4>::Floats);
}

constexpr int kMaxWaves = 8;   // n-tiles per block: dqk <= 128
constexpr int kKtStride = 20;  // floats per row of a wave's K transpose tile
constexpr int kStages = 4;   // deepest DMA ring
constexpr size_t kLdsBudget = 160 * 1024;
// sequences of fewer chunks stay whole (the fold pass would cost more than it saves)
constexpr int kMinSplitChunks = 64;
constexpr int kMinSplitChunksRank1 = 256;
constexpr int kFoldStages = 8;       // deepest DMA ring of the fold pass

// CUs of the current device (0 if unknown), looked up once per device.
int device_cus() {
  constexpr int kMaxDevices = 64;
  static std::atomic<int> cache[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return 0;
  int n = cache[dev].load(std::memory_order_relaxed);
  if (n > 0) return n;
  if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
    return 0;
  cache[dev].store(n, std::memory_order_relaxed);
  return n;
}

struct M3K {
  const float *q, *k, *v, *qb, *kb, *cos, *sin, *D, *z, *psi, *zeta, *phi;
  const float *adt, *dt, *trap;
  float *out, *last_state, *last_bx, *rec;
  int heads, dv, dqk, len, groups, nparts, nchunks, steps_per_chunk, nseq;
  int out_tm;  // out (b, l, h, dv) instead of (b, h, l, dv)
  int ptiles, nstages;
  int zown;  // z's step stride differs from v's (m3_chunk_kernel<.., ZOWN>)
  // DMA instructions (1 KB each) per stage: q and k take one per n-tile
  int n_cs, n_v, n_z;  // cos (and again sin), v, z
  int n_ins;           // all sections, + 2 for the gate record
  int stage_floats;
  // the fused angle pre-pass (m3_chunk_kernel<.., ANG>): raw angles (b, l, h, nang)
  // replace cos/sin (n_cs = 0) in n_ang DMA instructions per stage
  const float* ang;
  int nang, n_ang;
  int rec_floats;  // Rec<R>::Floats, or Rec<R>::FloatsAng with pi * dt per row
  long long vb, zb, ab, ah;  // element strides: v, z per batch; angles per batch, head
  int vt, zt, at;            // and per step
  // SISO: no same-step term (gamma on M's diagonal, D x) and out += the result
  int accum;
  // Sequences cut at chunk `split` (0: whole sequences): blocks [0, seg_blocks) run
  // chunks [split, nchunks) from the state m3_fold_kernel left in `fold`,
  // blocks [seg_blocks, 2 seg_blocks) run chunks [0, split) from zero.
  int split, seg_blocks;
  float* fold;
  int skip_q;  // the stage holds no q section (m3_fold_kernel's): k's comes first
  // The fold runs in nsub pieces of sub_len chunks, one block each (per sequence and dv
  // slices): piece s leaves its state from zero in fold + s * nseq * dv * dqk (in the
  // order the waves hold it, fold_off) and its decay (the product of its chunks'
  // e^{c_last}) in fold_decay[s * nseq + seq]; the resuming blocks combine them in order.
  int nsub, sub_len;
  float* fold_decay;
  // With the fused angle pre-pass (SISO): fold piece s rotates its keys by theta
  // relative to its first step and leaves theta's increment over its steps (turns,
  // reduced to [-1/2, 1/2]) per angle pair, 64 per sequence, at
  // theta[(s * nseq + seq) * 64 + pair]. Rotations compose, so its state equals the
  // true one times the rotation by theta at the piece's start (the increments of the
  // pieces before it), which the resuming blocks apply to the state's key columns.
  float* theta;
};

// ---------------------------------------------------------------------------
// Gate pre-pass: one lane per step, T = 16/R lanes per (sequence, chunk), a 16-lane
// group holding R chunks. Traversal step g maps to memory t = g (forward) or L-1-g
// (reverse); the trapezoid's "next" step is traversal step g+1 (mamba3/scalar.rs:95-115),
// absent at the end.
template <int R>
__global__ void __launch_bounds__(256) m3_gates_kernel(M3K p, int reverse) {
  using RC = Rec<R>;
  constexpr int T = RC::T;
  const int step = threadIdx.x & (T - 1);
  const long long nrec = (long long)p.nseq * p.nchunks;
  const int slot = threadIdx.x / T;  // the block's record of this lane
  const long long cidx = (long long)blockIdx.x * (256 / T) + slot;
  const bool valid = cidx < nrec;
  const int L = p.len;
  int seq = 0, ch = 0;
  if (valid) {
    seq = (int)(cidx / p.nchunks);
    ch = (int)(cidx - (long long)seq * p.nchunks);
  }
  const long long g = (long long)ch * T + step;
  float a = 0.0f, gamma = 0.0f, scale = 0.0f, hdt = 0.0f;
  if (valid && g < L) {
    const long long base = (long long)seq * L;  // gates are (b, h, l): seq = b*heads + h
    const long long t = reverse ? L - 1 - g : g;
    a = p.adt[base + t];
    hdt = 0.5f * p.dt[base + t];  // pi * dt radians in turns (exact)
    gamma = p.dt[base + t] * sigmoid(p.trap[base + t]);
    scale = gamma;
    if (g + 1 < L) {
      const long long tn = reverse ? t - 1 : t + 1;
      scale = gamma + p.dt[base + tn] * (1.0f - sigmoid(p.trap[base + tn]));
    }
  }
  // c_i: inclusive sum of adt over the chunk's steps up to i
  float c = a;
#pragma unroll
  for (int d = 1; d < T; d <<= 1) {
    const float o = __shfl_up(c, d, T);
    if (step >= d) c += o;
  }
  const float clast = __shfl(c, T - 1, T);
  float m[T];
#pragma unroll
  for (int s = 0; s < T; ++s) {
    const float cs = __shfl(c, s, T);
    const float ss = __shfl(scale, s, T);
    m[s] = s < step ? fexp(c - cs) * ss : (s == step && !p.accum ? gamma : 0.0f);
  }
  // The block's 256/T records are assembled in LDS and leave as one contiguous run of
  // 16-byte stores (written in place, a store instruction put 16 bytes into each of
  // 64 rows 64 bytes apart at rank 1).
  __shared__ __attribute__((aligned(16))) float img[(256 / T) * RC::FloatsAng];
  float* rec = img + slot * p.rec_floats;
  if (p.rec_floats > RC::Floats) {  // 0 past the end: theta holds
#pragma unroll
    for (int r = 0; r < R; ++r) rec[RC::Hdt + step * R + r] = hdt;  // the step's R rows
  }
  if constexpr (R == 1) {
    // row i's 16-byte pieces rotated by i/2 (piece q at (q + i/2) & 3): the scan's
    // epilogue reads a piece per lane, rows 64 bytes (16 banks) apart, and rotated the
    // eight lanes of a 128-byte read phase meet no bank conflict
    f4* mrow = reinterpret_cast<f4*>(rec + RC::M + step * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q)
      mrow[(q + (step >> 1)) & 3] = f4{m[4 * q], m[4 * q + 1], m[4 * q + 2], m[4 * q + 3]};
  } else {
#pragma unroll
    for (int q = 0; q < T; ++q) rec[RC::M + step * T + q] = m[q];
  }
  rec[RC::Ec + step] = fexp(c);
  rec[RC::W + step] = fexp(clast - c) * scale;
  // e^{c_last}, then zeros to the end of the last 16-byte piece
  static_assert(RC::Floats - RC::Etot <= T, "the padding fits the chunk's lanes");
  if (step < RC::Floats - RC::Etot) rec[RC::Etot + step] = step == 0 ? fexp(clast) : 0.0f;
  __syncthreads();
  const long long first = (long long)blockIdx.x * (256 / T);
  const long long left = nrec - first;
  const int n4 = (int)(left < 256 / T ? left : 256 / T) * p.rec_floats / 4;  // rec_floats % 4 == 0
  const f4* src = reinterpret_cast<const f4*>(img);
  f4* dst = reinterpret_cast<f4*>(p.rec + first * p.rec_floats);
  for (int i = threadIdx.x; i < n4; i += 256) dst[i] = src[i];
}

// ---------------------------------------------------------------------------
// Waits until at most N vector-memory operations of this wave are outstanding and
// every LDS operation of this wave is done. Vector memory operations complete in
// issue order on gfx9, so "at most N outstanding" means "all but the last N done".
template <int N>
__device__ __forceinline__ void waitcnt_vm() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | (7 << 4));  // lgkmcnt(0)
}

// The same for a run-time n, rounded down to a step of the ladder (waiting for
// more operations than needed is always safe).
__device__ __forceinline__ void wait_vm_at_most(int n) {
  if (n >= 16) waitcnt_vm<16>();
  else if (n >= 12) waitcnt_vm<12>();
  else if (n >= 8) waitcnt_vm<8>();
  else if (n >= 6) waitcnt_vm<6>();
  else if (n >= 4) waitcnt_vm<4>();
  else if (n >= 3) waitcnt_vm<3>();
  else if (n >= 2) waitcnt_vm<2>();
  else if (n >= 1) waitcnt_vm<1>();
  else waitcnt_vm<0>();
}

// Workgroup barrier that orders LDS only: outstanding global loads and stores
// stay in flight.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ f4 ld4(const float* p) { return *reinterpret_cast<const f4*>(p); }
__device__ __forceinline__ f2 ld2(const float* p) { return *reinterpret_cast<const f2*>(p); }

// A fold piece's state (dv x dqk per sequence) in the order the waves hold it: the
// 16-byte unit of lane `lane` of n-tile wave nt for the 16-column dv slice `slice`
// (rows slice*16 + lane%16, columns nt*16 + 4(lane/16) .. +3) at this float offset, so
// that a wave stores and loads a slice as one contiguous 1 KB run. In (seq, dv, dqk)
// order each store put 64 bytes into each of 16 rows 512 bytes apart.
__device__ __forceinline__ long long fold_off(int seq, int slice, int nt, int lane, int dv,
                                              int wn) {
  return ((((long long)seq * (dv / 16) + slice) * wn + nt) * 64 + lane) * 4;
}

// Base pointers of a block's sequence.
struct SeqIn {
  const float *q, *k, *cos, *sin, *ang, *v, *z, *rec;
  int qstride, csstride, angstride, vstride, zstride;  // floats per step
};

// DMA instruction `ins` of a stage (1 KB, one 16-byte piece per lane). Stage
// layout in pieces, each section padded to whole instructions:
//   q, k: piece (nt, lj, li) = columns nt*16 + 4lj .. +3 of row li
//   cos, sin: piece u4*T + step = angles 4u4 .. 4u4+3 of the step
//   or, fused, the raw angles: piece u4*T + step = angles 4u4 .. 4u4+3 of the step
//   v, z: piece step*4PT + c4 = columns p0 + 4c4 .. +3 of the step
//   gate record: its 73 pieces in order
// The lane's piece of chunk ch is src + t*stride + col with t the memory row of
// step `step` of the chunk, or src + ch*rec_floats + col for the gate record.
struct DmaPiece {
  const float* src;
  int step, col, stride;
  bool on, rec;
};

// The v and z sections of a stage hold step s's w4 = 4PT pieces rotated by four of them
// (16 floats, half the banks) when bits 0 and 2 of s differ: the 16-lane reads of steps
// s and s+1 (the partial waves' w x) and of s and s+4 (the epilogue waves' x and z), a
// slice of 16 columns each, by one 32-lane half then fall in different banks instead of
// on the same ones a multiple of 128 bytes apart. With one slice (w4 = 4) a read covers
// the whole 64-byte step, and no rotation within it changes its banks. Float offset of
// (step s, column c) in such a section; the DMA fills it through the inverse map.
__device__ __forceinline__ int vrot(int s, int w4) {
  return w4 >= 8 ? ((s ^ (s >> 2)) & 1) * 4 : 0;
}
__device__ __forceinline__ int vpos(int s, int c, int w4) {
  return s * 4 * w4 + 4 * (((c >> 2) + vrot(s, w4)) & (w4 - 1)) + (c & 3);
}

template <int R>
__device__ __forceinline__ DmaPiece dma_decode(const M3K& p, const SeqIn& s, int ins, int lane) {
  const int WN = p.dqk / 16, T = p.steps_per_chunk;
  DmaPiece d;
  d.step = 0;
  d.stride = 0;
  d.on = true;
  d.rec = false;
  int rel = ins;
  const int nq = p.skip_q ? 0 : WN;  // q's instructions
  if (rel < nq + WN) {
    const bool isq = rel < nq;
    const int nt = isq ? rel : rel - nq;
    const int li = lane & 15, lj = lane >> 4;
    d.src = isq ? s.q : s.k;
    d.step = li / R;
    d.col = (li % R) * p.groups * p.dqk + nt * 16 + 4 * lj;
    d.stride = s.qstride;
  } else if ((rel -= nq + WN) < 2 * p.n_cs) {
    const bool sn = rel >= p.n_cs;
    const int j = (sn ? rel - p.n_cs : rel) * 64 + lane;
    d.on = j < T * (p.dqk / 8);
    d.src = sn ? s.sin : s.cos;
    d.step = j % T;
    d.col = 4 * (j / T);
    d.stride = s.csstride;
  } else if ((rel -= 2 * p.n_cs) < p.n_ang) {
    const int j = rel * 64 + lane;
    d.on = j < T * (p.nang / 4);
    d.src = s.ang;
    d.step = j % T;
    d.col = 4 * (j / T);
    d.stride = s.angstride;
  } else if ((rel -= p.n_ang) < p.n_v + p.n_z) {
    const bool zz = rel >= p.n_v;
    const int j = (zz ? rel - p.n_v : rel) * 64 + lane;
    const int w4 = 4 * p.ptiles;
    d.on = j < T * w4;
    d.src = zz ? s.z : s.v;
    d.step = j / w4;
    d.col = 4 * (((j % w4) - vrot(d.step, w4)) & (w4 - 1));  // slot j % w4 holds that piece
    d.stride = zz ? s.zstride : s.vstride;
  } else {
    const int j = (rel - p.n_v - p.n_z) * 64 + lane;
    d.on = j < p.rec_floats / 4;
    d.src = s.rec;
    d.col = 4 * j;
    d.rec = true;
  }
  return d;
}

__device__ __forceinline__ void dma16(const float* src, float* lds) {
  __builtin_amdgcn_global_load_lds((const void*)src,
                                   (__attribute__((address_space(3))) void*)lds, 16, 0, 0);
}

// The DMA instructions of one wave, resolved once. For a chunk wholly inside the
// sequence the lane's source is base[k] + ch * delta[k] + off[k] (floats; base and
// delta are wave-uniform); the last, partial chunk goes through dma_clamped. A plan
// holds MD instructions: kNarrowDma when a stage needs no more than that per partial
// wave (dqk 128 at configs 3 and 4), else kMaxDma. The plan's scalars stay live
// through the chunk loop, in a kernel whose scalar registers spill: the narrow plan
// spills 222 SGPRs instead of 588 and runs configs 3 and 4 about 4% faster.
constexpr int kMaxDma = 8;
constexpr int kNarrowDma = 4;
template <int MD>
struct DmaPlan {
  const float* base[MD];
  int delta[MD];
  int off[MD];
  bool on[MD];
  int ins[MD];
  int count;
};

template <int R, bool REV, int MD>
__device__ __forceinline__ void dma_plan(const M3K& p, const SeqIn& s, int first, int step_ins,
                                         int lane, DmaPlan<MD>& d) {
  const int T = p.steps_per_chunk, L = p.len;
  d.count = 0;
#pragma unroll
  for (int k = 0; k < MD; ++k) {
    const int ins = first + k * step_ins;
    d.ins[k] = ins;
    d.on[k] = false;
    d.base[k] = s.rec;
    d.delta[k] = 0;
    d.off[k] = 0;
    if (ins < p.n_ins) {
      const DmaPiece pc = dma_decode<R>(p, s, ins, lane);
      d.count = k + 1;
      d.on[k] = pc.on;
      if (pc.rec) {
        d.base[k] = pc.src;
        d.delta[k] = p.rec_floats;
        d.off[k] = pc.col;
      } else if (!REV) {
        d.base[k] = pc.src;
        d.delta[k] = T * pc.stride;
        d.off[k] = pc.step * pc.stride + pc.col;
      } else {
        d.base[k] = pc.src + (long long)(L - 1) * pc.stride;
        d.delta[k] = -T * pc.stride;
        d.off[k] = pc.col - pc.step * pc.stride;
      }
    }
  }
}

// Any chunk, with the rows past the end clamped to the last step.
template <int R, bool REV, int MD>
__device__ __forceinline__ void dma_clamped(const M3K& p, const SeqIn& s, const DmaPlan<MD>& d,
                                            int ch, float* stage, int lane) {
  const int T = p.steps_per_chunk, L = p.len;
#pragma unroll
  for (int k = 0; k < MD; ++k) {
    if (k >= d.count) break;
    const DmaPiece pc = dma_decode<R>(p, s, d.ins[k], lane);
    if (!pc.on) continue;
    int g = ch * T + pc.step;
    g = g < L - 1 ? g : L - 1;
    const int t = REV ? L - 1 - g : g;
    const long long o = pc.rec ? (long long)ch * p.rec_floats + pc.col
                               : (long long)t * pc.stride + pc.col;
    dma16(pc.src + o, stage + d.ins[k] * 256);
  }
}

// The plan of a wave for whole chunks, as running pointers: instruction k of a stage
// reads ptr[k] + off[k] (the lane's piece) into stage + lds[k], and ptr[k] then moves
// on by one chunk (step[k] floats). A lane whose piece lies past its section's end
// (`on` false) reads the instruction's first piece into the section's padding, which
// nothing reads.
template <int MD>
struct DmaRun {
  const float* ptr[MD];
  int step[MD];
  int off[MD];
  int lds[MD];
  int count;
};

template <int MD>
__device__ __forceinline__ void dma_run(const DmaPlan<MD>& d, DmaRun<MD>& r, int first_chunk) {
  r.count = d.count;
#pragma unroll
  for (int k = 0; k < MD; ++k) {
    r.ptr[k] = d.base[k] + (long long)first_chunk * d.delta[k];
    r.step[k] = d.delta[k];
    r.off[k] = d.on[k] ? d.off[k] : 0;
    r.lds[k] = d.ins[k] * 256;
  }
}

// Instructions k0 .. k1-1 of the next whole chunk. CNT: the plan's instruction count
// when known at compile time (no per-instruction branch), else -1 (r.count).
template <int MD, int CNT = -1>
__device__ __forceinline__ void dma_part(DmaRun<MD>& r, float* stage, int k0, int k1) {
#pragma unroll
  for (int k = 0; k < MD; ++k) {
    if (k >= k0 && k < k1 && (CNT >= 0 ? k < CNT : k < r.count)) {
      dma16(r.ptr[k] + r.off[k], stage + r.lds[k]);
      r.ptr[k] += r.step[k];
    }
  }
}

template <int MD>
__device__ __forceinline__ void dma_next(DmaRun<MD>& r, float* stage) {
  dma_part(r, stage, 0, MD);
}

// Rotated q/k from the raw columns: SISO rotates interleaved pairs (2u, 2u+1)
// with angle u (mamba3/scalar.rs:40-48); MIMO rotates split halves (u, u + dqk/2)
// with angle u (mimo.rs:83-96), the lane holding its 4 columns x and their
// partners y.
template <bool MIMO>
__device__ __forceinline__ f4 rope(f4 x, f4 y, f4 bx, f4 by, f4 c, f4 s, bool lo) {
  x += bx;
  if (!MIMO)
    return f4{x[0] * c[0] - x[1] * s[0], x[0] * s[0] + x[1] * c[0],
              x[2] * c[1] - x[3] * s[1], x[2] * s[1] + x[3] * c[1]};
  y += by;
  return lo ? f4{x[0] * c[0] - y[0] * s[0], x[1] * c[1] - y[1] * s[1],
                 x[2] * c[2] - y[2] * s[2], x[3] * c[3] - y[3] * s[3]}
            : f4{y[0] * s[0] + x[0] * c[0], y[1] * s[1] + x[1] * c[1],
                 y[2] * s[2] + x[2] * c[2], y[3] * s[3] + x[3] * c[3]};
}

// tanh(a) = 1 - 2 / (1 + e^{2a}); saturates to +-1 through e^{2a} = inf or 0.
__device__ __forceinline__ float tanh_fast(float a) {
  return 1.0f - 2.0f * __builtin_amdgcn_rcpf(1.0f + fexp(2.0f * a));
}

// The angle pre-pass fused (python/arm_scan/mamba3.py:41-89: theta =
// cumsum_l(tanh(angle) * pi * dt), then cos/sin), for NA rotation pairs of the
// lane at row li of the chunk, in turns (theta / 2pi): hdt = dt / 2 is pi * dt
// radians in turns. The increments of rows li - R, li - 2R, .. (the earlier
// steps, same rank) are summed by a DPP row scan and added to the chunk's start
// angle `carry`; the sum is reduced to [-1/2, 1/2] turns, where cos/sin by the
// hardware functions of turns are exact to a few ulp, and the reduced angle at
// the chunk's last step carries on. The carry never grows: every add rounds at
// ulp(1/2) (3e-8 turns), where a running theta in radians rounds at ulp(theta)
// (1.5e-5 rad near 225 rad, the end of a sequence of one-signed angles at L 4096).
// All 64 lanes take part (the row scan and the carry's shuffle).
template <int R, int NA>
__device__ __forceinline__ void fused_angles(const float (&a)[NA], float hdt, int li,
                                             int lane, float (&carry)[NA], float (&cs)[NA],
                                             float (&sn)[NA]) {
#pragma unroll
  for (int e = 0; e < NA; ++e) {
    float t = tanh_fast(a[e]) * hdt;
    if (R <= 1) t += dpp<kRowShr1, 0xF>(0.0f, t);
    if (R <= 2) t += dpp<kRowShr2, 0xF>(0.0f, t);
    if (R <= 4) t += dpp<kRowShr4, 0xF>(0.0f, t);
    t += dpp<kRowShr8, 0xF>(0.0f, t);
    const float x = carry[e] + t;  // turns
    const float f = x - __builtin_rintf(x);
    carry[e] = __shfl(f, (lane & ~15) | (16 - R + li % R));
    cs[e] = __builtin_amdgcn_cosf(f);
    sn[e] = __builtin_amdgcn_sinf(f);
  }
}

// What a chunk's epilogue needs from its stage, kept in registers so that the
// stage can be refilled before the epilogue runs.
struct Stash {
  f4 m;   // M[li][4lj + r]
  f4 ec;  // e^{c} of rows 4lj + r
  f4 x;   // x of rows 4lj + r, in the wave's slice
  float z[4];
};

// Waves 0 .. WN-1 compute the partials of n-tile `wave` for every slice of the
// block; waves WN .. WN+2PT-1 finish slice (wave-WN) % PT of the chunks of parity
// (wave-WN) / PT. Both kinds pass one barrier per chunk.
// ACC: an accumulating traversal (p.accum; SISO without angles), a template parameter
// so that the other kernels carry none of its epilogue work. ZOWN: z's step stride
// differs from v's; otherwise z's DMA pieces share v's per-chunk step, one scalar
// fewer per piece in a kernel whose scalar registers already spill (measured 6%
// slower at config 3 with the two strides kept apart).
template <int R, bool MIMO, bool REV, int PT, bool ANG, bool ACC = false, bool ZOWN = false,
          int MD = kMaxDma>
__global__ void __launch_bounds__(64 * (kMaxWaves + 4)) m3_chunk_kernel(M3K p) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int WN = p.dqk / 16;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const bool ewave = wave >= WN;                    // epilogue wave
  // n-tile of a partial wave. MIMO with fused angles interleaves the halves (wave
  // 2i: n-tile i, 2i+1: WN/2 + i): the n-tiles holding the angle pairs below nang
  // then sit on different SIMDs (waves go to SIMDs round-robin).
  const int nt = ewave ? 0
                       : (MIMO && ANG && WN % 2 == 0)
                             ? ((wave & 1) ? WN / 2 + (wave >> 1) : (wave >> 1))
                             : wave;
  // epilogue waves: two per slice, taking the chunks of one parity each; a chunk's
  // epilogue spans two barrier intervals (reduce, then MFMA and store), so in every
  // interval the reductions of one parity and the finishing of the other run on
  // different SIMDs
  const int ej = ewave ? (wave - WN) % PT : 0;      // slice of an epilogue wave
  const int epar = ewave ? (wave - WN) / PT : 0;    // chunk parity of an epilogue wave
  const int li = lane & 15, lj = lane >> 4;
  // this block's chunks [cb, ce): the tail segment (from the folded state) comes first
  // in block order, so that its longer blocks start first; the head segment's blocks
  // fill the CUs left over, several in turn
  int bid = blockIdx.x, cb = 0, ce = p.nchunks;
  if (p.split) {
    if (bid >= p.seg_blocks) {
      bid -= p.seg_blocks;
      ce = p.split;
    } else {
      cb = p.split;
    }
  }
  // blocks of one sequence share an XCD (block id mod 8), and so its L2
  const int bx = bid & 7, by = bid >> 3;
  const int nb = p.nparts / PT;  // blocks per sequence
  const int seq = (by / nb) * 8 + bx;
  const int p0 = (by % nb) * PT * 16;  // first dv column of the block
  if (seq >= p.nseq) return;  // whole block exits: no barrier is reached by anyone
  const int H = p.heads;
  const int bi = seq / H, h = seq - bi * H;
  const int grp = h / (H / p.groups);
  const int L = p.len, dqk = p.dqk, dv = p.dv, T = p.steps_per_chunk, NS = p.nstages;
  const int half = dqk / 2;
  const int n0 = nt * 16 + 4 * lj;  // a partial wave's 4 columns of dqk
  const bool lo = !MIMO || n0 < half;
  const int step_i = li / R;

  // partials of every n-tile slot; the slots of absent n-tiles (WN < kMaxWaves) stay 0
  float* stages = sm;
  float* gbuf = stages + NS * p.stage_floats;  // [2][kMaxWaves][64][4]
  float* ybuf = gbuf + 2 * kMaxWaves * 256;     // [2][PT][kMaxWaves][64][4]
  constexpr bool KQ = !MIMO;  // K transposed in the stage's q piece (SISO)
  float* kt = ybuf + 2 * PT * kMaxWaves * 256 + nt * 16 * kKtStride;  // MIMO only
  const int off_k = WN * 256, off_cs = 2 * WN * 256;
  const int off_sn = off_cs + p.n_cs * 256, off_ang = off_cs + 2 * p.n_cs * 256;
  const int off_v = off_ang + p.n_ang * 256;
  const int off_z = off_v + p.n_v * 256, off_rec = off_z + p.n_z * 256;

  if (WN < kMaxWaves) {
    const f4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int e = threadIdx.x; e < 2 * (1 + PT) * kMaxWaves * 64; e += blockDim.x) {
      const int slot = (e >> 6) % kMaxWaves;
      if (slot >= WN) *reinterpret_cast<f4*>(gbuf + e * 4) = zero;  // ybuf follows gbuf
    }
  }

  if (ewave) {
    // ================= epilogue wave: slice ej =================
    const float dskip = p.D && !ACC ? p.D[h] : 0.0f;
    const int pcol = p0 + ej * 16 + li;
    float psi[4], zeta[4], phi[4];
#pragma unroll
    for (int m = 0; m < 4; ++m) {
      const long long pj = ((long long)h * R + (4 * lj + m) % R) * dv + pcol;
      psi[m] = MIMO ? p.psi[pj] : 1.0f;
      zeta[m] = (MIMO && p.z) ? p.zeta[pj] : 1.0f;
      phi[m] = MIMO ? p.phi[pj] : 1.0f;
    }
    // output of the lane's first row in chunk 0; ostep floats per step
    const int t0 = REV ? L - 1 - lj * 4 / R : lj * 4 / R;
    const int ostep = p.out_tm ? H * dv : dv;
    float* out_lane = p.out + pcol +
                      (p.out_tm ? (((long long)bi * L + t0) * H + h) * dv
                                : (((long long)bi * H + h) * L + t0) * dv);
    Stash st = {};
    const bool has_z = p.z != nullptr;
    const int sfl = p.stage_floats;
    const long long chstep = (REV ? -(long long)T : (long long)T) * ostep;  // per chunk
    // part A of chunk ch: the partials reduced and masked (lane: G[li][4lj + r] and the
    // inter-chunk Y[4lj + r][p]); it reads the partial buffers right after the
    // barrier that publishes them
    f4 G = {0.0f, 0.0f, 0.0f, 0.0f}, Y = {0.0f, 0.0f, 0.0f, 0.0f};
    // ACC: the output rows chunk ch adds to, loaded in its part A so that part B, an
    // interval later, does not wait for them before its stores
    float accp[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    auto part_a = [&](int ch) {
      if constexpr (ACC) {
        const float* orow = out_lane + (long long)ch * chstep;
#pragma unroll
        for (int r = 0; r < 4; r += R)
          if (ch * T + (4 * lj + r) / R < L) accp[r] = orow[(REV ? -(r / R) : r / R) * ostep];
      }
      const float* gb = gbuf + (ch & 1) * kMaxWaves * 256;
      const float* yb = ybuf + ((ch & 1) * PT + ej) * kMaxWaves * 256;
      f4 gs[kMaxWaves], ys[kMaxWaves];  // all reads in flight at once
#pragma unroll
      for (int w2 = 0; w2 < kMaxWaves; ++w2) {
        gs[w2] = ld4(gb + (w2 * 64 + lane) * 4);
        ys[w2] = ld4(yb + (w2 * 64 + lane) * 4);
      }
#pragma unroll
      for (int d = kMaxWaves / 2; d > 0; d /= 2)
#pragma unroll
        for (int w2 = 0; w2 < d; ++w2) {
          gs[w2] += gs[w2 + d];
          ys[w2] += ys[w2 + d];
        }
      G = gs[0] * st.m;
      Y = ys[0] * st.ec;
    };
    // part B of chunk ch: the intra-chunk term, D x, gating, rank sum, store.
    // FULL: every row of the chunk lies inside the sequence (all chunks but the last)
    auto part_b = [&](int ch, auto full) {
      constexpr bool FULL = decltype(full)::value;
      auto valid = [&](int r) { return FULL || ch * T + (4 * lj + r) / R < L; };
      float* orow = out_lane + (long long)ch * chstep;
      float prev[4] = {0.0f, 0.0f, 0.0f, 0.0f};
      if constexpr (ACC) {
#pragma unroll
        for (int r = 0; r < 4; r += R) prev[r] = accp[r];
      }
      f4 Yc = Y;
#pragma unroll
      for (int m = 0; m < 4; ++m) Yc = mfma(G[m], st.x[m], Yc);
#pragma unroll
      for (int r = 0; r < 4; r += R) {
        if (valid(r)) {
          float acc = prev[r];
#pragma unroll
          for (int rr = 0; rr < R; ++rr) {
            float term = Yc[r + rr] + dskip * st.x[r + rr];
            if (has_z) term *= silu_fast(st.z[r] * zeta[r + rr]);
            acc = fmaf(phi[r + rr], term, acc);
          }
          orow[(REV ? -(r / R) : r / R) * ostep] = acc;
        }
      }
    };
    // what the epilogue of a chunk needs from its stage
    auto stash = [&](const float* sg) {
      using RC = Rec<R>;
      if constexpr (R == 1) {
        st.m = ld4(sg + off_rec + RC::M + li * 16 + 4 * ((lj + (li >> 1)) & 3));
        st.ec = ld4(sg + off_rec + RC::Ec + 4 * lj);
      } else {  // rows 4lj + r lie in steps (4lj + r) / R
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          st.m[r] = sg[off_rec + RC::M + (li / R) * RC::T + (4 * lj + r) / R];
          st.ec[r] = sg[off_rec + RC::Ec + (4 * lj + r) / R];
        }
      }
#pragma unroll
      for (int m = 0; m < 4; ++m)
        st.x[m] = sg[off_v + vpos((4 * lj + m) / R, ej * 16 + li, 4 * PT)] * psi[m];
      if (has_z) {
#pragma unroll
        for (int r = 0; r < 4; r += R)
          st.z[r] = sg[off_z + vpos((4 * lj + r) / R, ej * 16 + li, 4 * PT)];
      }
    };
    // chunks cb .. ce-1 (parities by the absolute chunk index, as the partial waves
    // write them); the ring slot of chunk ch is (ch - cb) mod NS
    lds_barrier();  // stage of chunk cb landed
    if ((cb & 1) == epar) stash(stages);
    int slot = 0;
    for (int ch = cb + 1; ch < ce; ++ch) {
      slot = slot + 1 == NS ? 0 : slot + 1;
      lds_barrier();  // stage ch landed, partials of chunk ch-1 written
      const int c = ch - 1;
      if ((c & 1) == epar) part_a(c);
      else if (c > cb) part_b(c - 1, std::true_type{});  // this wave's previous chunk
      if ((ch & 1) == epar) stash(stages + slot * sfl);
    }
    lds_barrier();  // partials of the block's last chunk written
    const int cl = ce - 1;
    if ((cl & 1) == epar) {
      part_a(cl);
      part_b(cl, std::false_type{});
    } else if (cl > cb) {
      part_b(cl - 1, std::true_type{});
    }
    return;
  }

  // ================= partial wave: n-tile nt =================
  SeqIn in;
  in.q = p.q + ((long long)bi * L * R * p.groups + grp) * dqk;
  in.k = p.k + ((long long)bi * L * R * p.groups + grp) * dqk;
  in.cos = p.cos + ((long long)bi * L * H + h) * half;
  in.sin = p.sin + ((long long)bi * L * H + h) * half;
  in.v = p.v + (long long)bi * p.vb + (long long)h * dv + p0;
  in.z = p.z ? p.z + (long long)bi * p.zb + (long long)h * dv + p0 : nullptr;
  in.ang = ANG ? p.ang + (long long)bi * p.ab + (long long)h * p.ah : nullptr;
  in.rec = p.rec + (long long)seq * p.nchunks * p.rec_floats;
  in.qstride = R * p.groups * dqk;
  in.csstride = H * half;
  in.angstride = p.at;
  in.vstride = p.vt;
  in.zstride = ZOWN ? p.zt : p.vt;

  // biases of the lane's columns (row li has rank li % R)
  f4 bq, bk, bqp = {0.0f, 0.0f, 0.0f, 0.0f}, bkp = bqp;
  const int m0 = n0 < half ? n0 + half : n0 - half;  // MIMO partner columns
  {
    const long long bo = ((long long)h * R + (li % R)) * dqk;
    bq = ld4(p.qb + bo + n0);
    bk = ld4(p.kb + bo + n0);
    if (MIMO) {
      bqp = ld4(p.qb + bo + m0);
      bkp = ld4(p.kb + bo + m0);
    }
  }
  float psi[PT][4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int j = 0; j < PT; ++j)
      psi[j][m] = MIMO ? p.psi[((long long)h * R + (4 * lj + m) % R) * dv + p0 + j * 16 + li]
                       : 1.0f;

  // The DMA instructions of this wave; the partial waves issue no other vector
  // memory operation inside the loop. Full chunks go through the running pointers of
  // DmaRun, the last chunk (when partial) through dma_clamped.
  DmaPlan<MD> dp;
  dma_plan<R, REV>(p, in, nt, WN, lane, dp);
  DmaRun<MD> dr;
  dma_run(dp, dr, cb);
  const int nfull = L / T;  // chunks wholly inside the sequence
  const int sfl = p.stage_floats;
  // ring slot r holds chunk cb + r first
  for (int r = 0; r < NS - 1 && cb + r < ce; ++r) {
    if (cb + r < nfull) dma_next(dr, stages + r * sfl);
    else dma_clamped<R, REV>(p, in, dp, cb + r, stages + r * sfl, lane);
  }
  const int wait_n = (NS - 2) * dp.count;  // outstanding DMA allowed in the steady state

  // The state update of chunk c runs after the barrier of chunk c+1, from operands kept
  // in registers (K transposed, w x, e^{c_last}): the MFMA work it brings covers the LDS
  // latency of chunk c+1's q/k rows.
  f4 S[PT];
#pragma unroll
  for (int j = 0; j < PT; ++j) S[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  // fused angles: theta before the chunk of the pairs the lane computes (SISO: pairs
  // 8nt + 2lj + e)
  float carry[2] = {0.0f, 0.0f};       // SISO: 2 per lane
  // resuming at chunk cb = split: the head segment's state, its pieces in order, and
  // with fused angles theta there, the pieces' increments summed
  for (int sb = 0; cb > 0 && sb < p.nsub; ++sb) {
    const float dcy = p.fold_decay[sb * p.nseq + seq];
    const float* fold = p.fold + (long long)sb * p.nseq * dv * dqk;
    float c0 = 1.0f, s0 = 0.0f, c1 = 1.0f, s1 = 0.0f;
    if (ANG && !MIMO) {  // the piece's keys were rotated from its own start: rotate by
                         // theta there, the increments of the pieces before it
      c0 = __builtin_amdgcn_cosf(carry[0]);
      s0 = __builtin_amdgcn_sinf(carry[0]);
      c1 = __builtin_amdgcn_cosf(carry[1]);
      s1 = __builtin_amdgcn_sinf(carry[1]);
      const float* th = p.theta + ((long long)sb * p.nseq + seq) * 64 + 8 * nt + 2 * lj;
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        carry[e] += th[e];
        carry[e] -= __builtin_rintf(carry[e]);
      }
    }
#pragma unroll
    for (int j = 0; j < PT; ++j) {
      const f4 f = ld4(fold + fold_off(seq, p0 / 16 + j, nt, lane, dv, WN));
      const f4 r = ANG && !MIMO ? f4{f[0] * c0 - f[1] * s0, f[0] * s0 + f[1] * c0,
                                     f[2] * c1 - f[3] * s1, f[2] * s1 + f[3] * c1}
                                : f;
      S[j] = S[j] * dcy + r;
    }
  }
  float kc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 wx[PT];
#pragma unroll
  for (int j = 0; j < PT; ++j) wx[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float etot = 1.0f;
  f4 kr_last = {0.0f, 0.0f, 0.0f, 0.0f};
  float carry_m[4 / R] = {};           // MIMO: 4/R per lane
  float* gw = gbuf + (nt * 64 + lane) * 4;         // this wave's G partial, chunk parity 0
  float* yw = ybuf + (nt * 256 + lane * 4);        // its Y partials: + ((par * PT + j) * 8) * 256
  float* ktw = kt + li * kKtStride + 4 * lj;       // K transpose: written as rows
  const float* ktr = kt + 4 * lj * kKtStride + li; // read as columns
  int slot = 0;                                    // ring slot of chunk ch
  int dslot = NS - 1;                              // ring slot of chunk ch + NS - 1
  // One chunk. FAST: the chunk this iteration's DMA fetches lies wholly inside the
  // sequence, so the DMA is issued unconditionally and the compiler may schedule the
  // MFMA phases across it.
  // CNT: this wave's DMA instructions per stage when known at compile time, else -1;
  // WAIT: the steady state's vmcnt, (NS - 2) stages of them, when known, else -1 (a
  // run-time ladder). The steady-state loop below is instantiated for the common plans:
  // scalar branches per chunk (the ladder, a test per DMA instruction) slowed it, and the
  // compile-time vmcnt took configs 3 and 4 from 0.310 / 1.000 to 0.297 / 0.926 ms.
  auto chunk = [&](const int ch, auto fast, auto cnt_c, auto wait_c) {
    constexpr bool FAST = decltype(fast)::value;
    constexpr int CNT = decltype(cnt_c)::value;
    constexpr int WAIT = decltype(wait_c)::value;
    // Stage ch has landed once no more of this wave's DMA is outstanding than the
    // stages issued after it.
    if constexpr (FAST && WAIT >= 0) waitcnt_vm<WAIT>();
    else if (FAST || ch + NS - 2 < ce - 1) wait_vm_at_most(wait_n);
    else wait_vm_at_most((ce - 1 - ch) * dp.count);
    lds_barrier();
    const float* sg = stages + slot * sfl;
    float* dstage = stages + dslot * sfl;
    const int dch = ch + NS - 1;  // the chunk this iteration's DMA fetches
    const bool dma_fast_now = FAST || (dch < nfull && dch < ce);
    if (!FAST && dch >= nfull && dch < ce) dma_clamped<R, REV>(p, in, dp, dch, dstage, lane);

    // ---- q/k rows of this n-tile (LDS reads in flight during the state update)
    const f4 q = ld4(sg + (nt * 64 + lane) * 4);
    const f4 k = ld4(sg + off_k + (nt * 64 + lane) * 4);
    f4 qp = {0.0f, 0.0f, 0.0f, 0.0f}, kp = qp, cs, sn;
    if (MIMO) {
      const int pl = ((m0 >> 4) * 64 + ((m0 & 15) >> 2) * 16 + li) * 4;
      qp = ld4(sg + pl);
      kp = ld4(sg + off_k + pl);
    }
    if (!ANG) {
      if (MIMO) {
        const int u4 = (lo ? n0 : n0 - half) >> 2;
        cs = ld4(sg + off_cs + (u4 * T + step_i) * 4);
        sn = ld4(sg + off_sn + (u4 * T + step_i) * 4);
      } else {
        const int o = ((2 * nt + (lj >> 1)) * T + li) * 4 + 2 * (lj & 1);
        const f2 c2 = ld2(sg + off_cs + o), s2 = ld2(sg + off_sn + o);
        cs = f4{c2[0], c2[1], 0.0f, 0.0f};
        sn = f4{s2[0], s2[1], 0.0f, 0.0f};
      }
    }
    // ---- the deferred state update of chunk ch-1: S = e^{c_last} S + K^T diag(w) X
#pragma unroll
    for (int j = 0; j < PT; ++j) S[j] *= etot;
#pragma unroll
    for (int m = 0; m < 4; ++m)
#pragma unroll
      for (int j = 0; j < PT; ++j) S[j] = mfma(kc[m], wx[j][m], S[j]);
    if (dma_fast_now) dma_part<MD, FAST ? CNT : -1>(dr, dstage, 0, 1);
    // ---- rotated q/k rows
    if (ANG) {
      // pairs 4u4 .. 4u4+3 of the lane (MIMO) or 2 at 8nt + 2lj (SISO); past nang 0
      const int u4 = MIMO ? (lo ? n0 : n0 - half) >> 2 : 2 * nt + (lj >> 1);
      const bool have = 4 * u4 < p.nang;
      if ((MIMO ? (16 * nt) % half : 8 * nt) >= p.nang) {
        // every pair of the wave is past nang (wave-uniform): the identity rotation
        cs = f4{1.0f, 1.0f, 1.0f, 1.0f};
        sn = f4{0.0f, 0.0f, 0.0f, 0.0f};
      } else if (MIMO) {
        // the R lanes of a step (ranks) need the same four angles: each computes
        // 4/R of them, pair e = (li % R) * NC + c, and gathers the rest
        constexpr int NC = 4 / R;
        float a[NC], c[NC], sv[NC];
#pragma unroll
        for (int j = 0; j < NC; ++j)
          a[j] = have ? sg[off_ang + (u4 * T + step_i) * 4 + (li % R) * NC + j] : 0.0f;
        fused_angles<R, NC>(a, sg[off_rec + Rec<R>::Hdt + li], li, lane, carry_m, c, sv);
        const int src = lane - li % R;  // the step's first lane
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          cs[e] = NC == 4 ? c[e % NC] : __shfl(c[e % NC], src + e / NC);
          sn[e] = NC == 4 ? sv[e % NC] : __shfl(sv[e % NC], src + e / NC);
        }
      } else {
        float a[2], c[2], sv[2];
        const f2 a2 = have ? ld2(sg + off_ang + (u4 * T + li) * 4 + 2 * (lj & 1)) : f2{0, 0};
        a[0] = a2[0];
        a[1] = a2[1];
        fused_angles<R, 2>(a, sg[off_rec + Rec<R>::Hdt + li], li, lane, carry, c, sv);
        cs = f4{c[0], c[1], 0.0f, 0.0f};
        sn = f4{sv[0], sv[1], 0.0f, 0.0f};
      }
    }
    const f4 qr = rope<MIMO>(q, qp, bq, bqp, cs, sn, lo);
    const f4 kr = rope<MIMO>(k, kp, bk, bkp, cs, sn, lo);
    kr_last = kr;
    if (dma_fast_now) dma_part<MD, FAST ? CNT : -1>(dr, dstage, 1, 2);
    // ---- K transposed through LDS: the operand of this chunk's (deferred) state
    // update. SISO: in this wave's own q piece of the stage (read above; no other wave
    // reads it), rows of 16 floats, with the reduction index s = lj + 4m so that the
    // column reads meet no bank conflict. MIMO, whose partner pieces other waves read:
    // in a tile of the wave's own. The round trip and the reads of w x overlap the
    // MFMA chains below.
    // Row r's 16-byte pieces sit rotated by r/2 (piece c at 4 ((c + r/2) & 3)): rows are
    // 64 bytes, 16 banks, apart, so unrotated the eight lanes of a 128-byte write phase
    // (rows 0 .. 7 of one piece) would meet in two bank groups; rotated they cover all
    // eight, and the column reads stay conflict-free.
    float* const kq = stages + slot * sfl + nt * 256;
    *reinterpret_cast<f4*>(KQ ? kq + li * 16 + 4 * ((lj + (li >> 1)) & 3) : ktw) = kr;
#pragma unroll
    for (int m = 0; m < 4; ++m)
      kc[m] = KQ ? kq[(lj + 4 * m) * 16 + 4 * (((li >> 2) + (lj >> 1) + 2 * m) & 3) + (li & 3)]
                 : ktr[m * kKtStride];
    {
      f4 w;
      if (KQ) {  // SISO: rows lj + 4m
#pragma unroll
        for (int m = 0; m < 4; ++m) w[m] = sg[off_rec + Rec<R>::W + lj + 4 * m];
      } else if (R == 1) {
        w = ld4(sg + off_rec + Rec<R>::W + 4 * lj);
      } else {  // rows 4lj + m lie in steps (4lj + m) / R
#pragma unroll
        for (int m = 0; m < 4; ++m) w[m] = sg[off_rec + Rec<R>::W + (4 * lj + m) / R];
      }
      etot = sg[off_rec + Rec<R>::Etot];
#pragma unroll
      for (int j = 0; j < PT; ++j)
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int srow = KQ ? lj + 4 * m : (4 * lj + m) / R;  // the step of row s
          wx[j][m] = w[m] * (sg[off_v + vpos(srow, j * 16 + li, 4 * PT)] * psi[j][m]);
        }
    }
    // ---- partial G^T, and partial Q S0^T per slice: 1 + PT chains, interleaved
    const int par = ch & 1;
    f4 gp = {0.0f, 0.0f, 0.0f, 0.0f};
    f4 yp[PT];
#pragma unroll
    for (int j = 0; j < PT; ++j) yp[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      gp = mfma(kr[r], qr[r], gp);
#pragma unroll
      for (int j = 0; j < PT; ++j) yp[j] = mfma(qr[r], S[j][r], yp[j]);
    }
    if (dma_fast_now) dma_part<MD, FAST ? CNT : -1>(dr, dstage, 2, 3);
    *reinterpret_cast<f4*>(gw + par * kMaxWaves * 256) = gp;
#pragma unroll
    for (int j = 0; j < PT; ++j)
      *reinterpret_cast<f4*>(yw + ((par * PT + j) * kMaxWaves) * 256) = yp[j];
    if (dma_fast_now) dma_part<MD, FAST ? CNT : -1>(dr, dstage, 3, MD);
    slot = slot + 1 == NS ? 0 : slot + 1;
    dslot = dslot + 1 == NS ? 0 : dslot + 1;
  };
  // chunks whose DMA target (NS-1 ahead) is a whole chunk of this block's range
  const int dend = nfull < ce ? nfull : ce;
  const int nmain = dend - (NS - 1);
  int ch = cb;
  using std::integral_constant;
  auto steady = [&](auto cnt_c, auto wait_c) {
    for (; ch < nmain; ++ch) chunk(ch, std::true_type{}, cnt_c, wait_c);
  };
  using I2 = integral_constant<int, 2>;
  using I3 = integral_constant<int, 3>;
  using I4 = integral_constant<int, 4>;
  using IX = integral_constant<int, -1>;
  // Rank 1 fixes the instruction count as well (config 3: 0.296 -> 0.293 ms); at rank 4
  // that schedule came out slower (config 4: 0.918 -> 0.959 ms), so it keeps the count a
  // run-time value. Both bit-identical.
  if constexpr (R == 1) {
    switch (NS * 16 + dp.count) {  // wave-uniform
      case 4 * 16 + 4: steady(I4{}, integral_constant<int, 8>{}); break;  // config 3, waves 0-3
      case 4 * 16 + 3: steady(I3{}, integral_constant<int, 6>{}); break;  // config 3, waves 4-7
      case 4 * 16 + 2: steady(I2{}, I4{}); break;
      case 3 * 16 + 4: steady(I4{}, I4{}); break;
      case 3 * 16 + 3: steady(I3{}, I3{}); break;
      case 3 * 16 + 2: steady(I2{}, I2{}); break;
      default: steady(IX{}, IX{}); break;
    }
  } else {
    switch (wait_n) {  // wave-uniform
      case 2: steady(IX{}, I2{}); break;
      case 3: steady(IX{}, I3{}); break;
      case 4: steady(IX{}, I4{}); break;                           // config 4, waves 4-7
      case 6: steady(IX{}, integral_constant<int, 6>{}); break;   // config 4, waves 0-3
      case 8: steady(IX{}, integral_constant<int, 8>{}); break;
      case 12: steady(IX{}, integral_constant<int, 12>{}); break;
      default: steady(IX{}, IX{}); break;
    }
  }
  for (; ch < ce; ++ch) chunk(ch, std::false_type{}, IX{}, IX{});
  // the last chunk's state update
#pragma unroll
  for (int j = 0; j < PT; ++j) S[j] *= etot;
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int j = 0; j < PT; ++j) S[j] = mfma(kc[m], wx[j][m], S[j]);
  lds_barrier();

  if (p.last_state && ce == p.nchunks) {
#pragma unroll
    for (int j = 0; j < PT; ++j)
      *reinterpret_cast<f4*>(p.last_state + ((long long)seq * dv + p0 + j * 16 + li) * dqk + n0) =
          S[j];
  }
  if (p.last_bx && p0 == 0 && ce == p.nchunks) {
    // scale k at the final step = k times the w of its row (the chunk's last valid row)
    const int last = p.nchunks - 1;
    if (li % R == 0 && last * T + step_i == L - 1) {
      const float* sg = stages + ((last - cb) % NS) * p.stage_floats;
      *reinterpret_cast<f4*>(p.last_bx + (long long)seq * dqk + n0) =
          kr_last * sg[off_rec + Rec<R>::W + li / R];
    }
  }
}

// The state a sequence reaches after its chunks [0, p.split), from zero, written to
// p.fold (in fold_off's order): the partial waves' state update alone (no q, no outputs, no
// epilogue waves), S = e^{c_last} S + K^T diag(w) X per chunk, for the blocks of
// m3_chunk_kernel that resume at chunk p.split. Its stage is the scan's without q and z
// (the host builds this kernel's M3K so: skip_q), about 20 KB at config 3, so that a
// ring of up to kFoldStages stages keeps 7 chunks of DMA in flight: the pass does little
// work per chunk, and with the scan's 3 chunks ahead it waited on memory. K is
// transposed through a per-wave tile, for SISO as for MIMO.
template <int R, bool MIMO, bool REV, int PT, int MD>
__global__ void __launch_bounds__(64 * kMaxWaves) m3_fold_kernel(M3K p) {
  extern __shared__ __attribute__((aligned(16))) float sm[];
  const int WN = p.dqk / 16;
  const int lane = threadIdx.x & 63;
  const int nt = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int li = lane & 15, lj = lane >> 4;
  const int sub = blockIdx.x / p.seg_blocks;  // this block's piece of the head segment
  const int bid = blockIdx.x - sub * p.seg_blocks;
  const int bx = bid & 7, by = bid >> 3;
  const int nb = p.nparts / PT;
  const int seq = (by / nb) * 8 + bx;
  const int p0 = (by % nb) * PT * 16;
  if (seq >= p.nseq) return;  // whole block: no barrier is reached
  const int H = p.heads;
  const int bi = seq / H, h = seq - bi * H;
  const int grp = h / (H / p.groups);
  const int L = p.len, dqk = p.dqk, dv = p.dv, T = p.steps_per_chunk, NS = p.nstages;
  const int half = dqk / 2;
  const int n0 = nt * 16 + 4 * lj;
  const bool lo = !MIMO || n0 < half;
  const int step_i = li / R;
  // chunks [cb, ce) of the head segment [0, split), all whole (split < L / T)
  const int cb = sub * p.sub_len;
  const int ce = cb + p.sub_len < p.split ? cb + p.sub_len : p.split;
  float* stages = sm;
  float* kt = stages + NS * p.stage_floats + nt * 16 * kKtStride;
  const int off_k = 0, off_cs = WN * 256;
  const int off_sn = off_cs + p.n_cs * 256, off_ang = off_cs + 2 * p.n_cs * 256;
  const int off_v = off_ang + p.n_ang * 256;
  const int off_rec = off_v + p.n_v * 256;
  // the fused angle pre-pass (SISO): the stage holds raw angles in place of cos/sin,
  // and theta enters the piece as the sum of the pieces before it
  const bool ang = !MIMO && p.ang != nullptr;

  SeqIn in;
  in.q = p.q + ((long long)bi * L * R * p.groups + grp) * dqk;
  in.k = p.k + ((long long)bi * L * R * p.groups + grp) * dqk;
  in.cos = p.cos + ((long long)bi * L * H + h) * half;
  in.sin = p.sin + ((long long)bi * L * H + h) * half;
  in.v = p.v + (long long)bi * p.vb + (long long)h * dv + p0;
  in.z = nullptr;
  in.ang = ang ? p.ang + (long long)bi * p.ab + (long long)h * p.ah : nullptr;
  in.rec = p.rec + (long long)seq * p.nchunks * p.rec_floats;
  in.qstride = R * p.groups * dqk;
  in.csstride = H * half;
  in.angstride = p.at;
  in.vstride = p.vt;
  in.zstride = p.vt;

  f4 bk, bkp = {0.0f, 0.0f, 0.0f, 0.0f};
  const int m0 = n0 < half ? n0 + half : n0 - half;  // MIMO partner columns
  {
    const long long bo = ((long long)h * R + (li % R)) * dqk;
    bk = ld4(p.kb + bo + n0);
    if (MIMO) bkp = ld4(p.kb + bo + m0);
  }
  float psi[PT][4];
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int j = 0; j < PT; ++j)
      psi[j][m] = MIMO ? p.psi[((long long)h * R + (4 * lj + m) % R) * dv + p0 + j * 16 + li]
                       : 1.0f;

  DmaPlan<MD> dp;
  dma_plan<R, REV>(p, in, nt, WN, lane, dp);
  DmaRun<MD> dr;
  dma_run(dp, dr, cb);
  const int sfl = p.stage_floats;
  // One stage of DMA per iteration, chunk ch + NS - 1 or, past the range, chunk ce - 1
  // again (into the slot of a chunk every wave has finished, which nothing reads), so
  // that behind the stage a wave waits for there are always NS - 2 of its stages in
  // flight: a vmcnt known at compile time (the loop below is instantiated per count)
  // in place of a run-time ladder of them, whose scalar branches cost more than the
  // chunk's work.
  auto issue = [&](float* stage, bool advance) {
#pragma unroll
    for (int k = 0; k < MD; ++k) {
      if (k < dr.count) {
        dma16(dr.ptr[k] + dr.off[k], stage + dr.lds[k]);
        if (advance) dr.ptr[k] += dr.step[k];
      }
    }
  };
  for (int r = 0; r < NS - 1; ++r) issue(stages + r * sfl, cb + r < ce - 1);

  f4 S[PT];
#pragma unroll
  for (int j = 0; j < PT; ++j) S[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float kc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  f4 wx[PT];
#pragma unroll
  for (int j = 0; j < PT; ++j) wx[j] = f4{0.0f, 0.0f, 0.0f, 0.0f};
  float etot = 1.0f, decay = 1.0f;
  // fused angles: theta before the chunk (SISO pairs 8nt + 2lj + e), relative to the
  // piece's first step
  float carry[2] = {0.0f, 0.0f};
  float* ktw = kt + li * kKtStride + 4 * lj;
  const float* ktr = kt + 4 * lj * kKtStride + li;
  auto run = [&](auto wcount) {
    constexpr int W = decltype(wcount)::value;
    int slot = 0, dslot = NS - 1;
    for (int ch = cb; ch < ce; ++ch) {
      waitcnt_vm<W>();
      lds_barrier();
      const float* sg = stages + slot * sfl;
      float* dstage = stages + dslot * sfl;
      const f4 k = ld4(sg + off_k + (nt * 64 + lane) * 4);
      f4 kp = {0.0f, 0.0f, 0.0f, 0.0f}, cs, sn;
      if (MIMO) {
        const int pl = ((m0 >> 4) * 64 + ((m0 & 15) >> 2) * 16 + li) * 4;
        kp = ld4(sg + off_k + pl);
        const int u4 = (lo ? n0 : n0 - half) >> 2;
        cs = ld4(sg + off_cs + (u4 * T + step_i) * 4);
        sn = ld4(sg + off_sn + (u4 * T + step_i) * 4);
      } else if (ang) {
        // pairs 8nt + 2lj, +1 (0 past nang); a wave whose pairs all lie past nang
        // (wave-uniform) takes the identity rotation, as the scan's does
        if (8 * nt >= p.nang) {
          cs = f4{1.0f, 1.0f, 0.0f, 0.0f};
          sn = f4{0.0f, 0.0f, 0.0f, 0.0f};
        } else {
          const int u4 = 2 * nt + (lj >> 1);
          const f2 a2 = 4 * u4 < p.nang ? ld2(sg + off_ang + (u4 * T + li) * 4 + 2 * (lj & 1))
                                        : f2{0.0f, 0.0f};
          float a[2] = {a2[0], a2[1]}, c[2], sv[2];
          fused_angles<R, 2>(a, sg[off_rec + Rec<R>::Hdt + li], li, lane, carry, c, sv);
          cs = f4{c[0], c[1], 0.0f, 0.0f};
          sn = f4{sv[0], sv[1], 0.0f, 0.0f};
        }
      } else {
        const int o = ((2 * nt + (lj >> 1)) * T + li) * 4 + 2 * (lj & 1);
        const f2 c2 = ld2(sg + off_cs + o), s2 = ld2(sg + off_sn + o);
        cs = f4{c2[0], c2[1], 0.0f, 0.0f};
        sn = f4{s2[0], s2[1], 0.0f, 0.0f};
      }
      // the deferred update of chunk ch-1
#pragma unroll
      for (int j = 0; j < PT; ++j) S[j] *= etot;
#pragma unroll
      for (int m = 0; m < 4; ++m)
#pragma unroll
        for (int j = 0; j < PT; ++j) S[j] = mfma(kc[m], wx[j][m], S[j]);
      issue(dstage, ch + NS - 1 < ce - 1);
      const f4 kr = rope<MIMO>(k, kp, bk, bkp, cs, sn, lo);
      // K transposed: reduction index s = 4lj + m (rows 4lj + m of the chunk)
      *reinterpret_cast<f4*>(ktw) = kr;
#pragma unroll
      for (int m = 0; m < 4; ++m) kc[m] = ktr[m * kKtStride];
      f4 w;
      if (R == 1) {
        w = ld4(sg + off_rec + Rec<R>::W + 4 * lj);
      } else {
#pragma unroll
        for (int m = 0; m < 4; ++m) w[m] = sg[off_rec + Rec<R>::W + (4 * lj + m) / R];
      }
      etot = sg[off_rec + Rec<R>::Etot];
      decay *= etot;
#pragma unroll
      for (int j = 0; j < PT; ++j)
#pragma unroll
        for (int m = 0; m < 4; ++m)
          wx[j][m] = w[m] * (sg[off_v + vpos((4 * lj + m) / R, j * 16 + li, 4 * PT)] * psi[j][m]);
      slot = slot + 1 == NS ? 0 : slot + 1;
      dslot = dslot + 1 == NS ? 0 : dslot + 1;
    }
  };
  using std::integral_constant;
  switch ((NS - 2) * dr.count) {  // wave-uniform
    case 1: run(integral_constant<int, 1>{}); break;
    case 2: run(integral_constant<int, 2>{}); break;
    case 3: run(integral_constant<int, 3>{}); break;
    case 4: run(integral_constant<int, 4>{}); break;
    case 5: run(integral_constant<int, 5>{}); break;
    case 6: run(integral_constant<int, 6>{}); break;
    case 8: run(integral_constant<int, 8>{}); break;
    case 9: run(integral_constant<int, 9>{}); break;
    case 10: run(integral_constant<int, 10>{}); break;
    case 12: run(integral_constant<int, 12>{}); break;
    case 15: run(integral_constant<int, 15>{}); break;
    case 18: run(integral_constant<int, 18>{}); break;
    default: run(integral_constant<int, 0>{}); break;  // waits for more: always safe
  }
  waitcnt_vm<0>();  // the re-fetches past the range land before the block's LDS is freed
#pragma unroll
  for (int j = 0; j < PT; ++j) S[j] *= etot;
#pragma unroll
  for (int m = 0; m < 4; ++m)
#pragma unroll
    for (int j = 0; j < PT; ++j) S[j] = mfma(kc[m], wx[j][m], S[j]);
  float* fold = p.fold + (long long)sub * p.nseq * dv * dqk;
#pragma unroll
  for (int j = 0; j < PT; ++j)
    *reinterpret_cast<f4*>(fold + fold_off(seq, p0 / 16 + j, nt, lane, dv, WN)) = S[j];
  if (p0 == 0 && nt == 0 && lane == 0) p.fold_decay[sub * p.nseq + seq] = decay;
  if (ang && p0 == 0 && li == 0) {  // theta's increment over the piece (0 past nang)
    float* th = p.theta + ((long long)sub * p.nseq + seq) * 64 + 8 * nt + 2 * lj;
    th[0] = carry[0];
    th[1] = carry[1];
  }
}

size_t chunk_lds_bytes(const M3K& k, int pt, int ns) {
  const int WN = k.dqk / 16;
  const size_t kt = k.psi ? (size_t)WN * 16 * kKtStride : 0;  // SISO: in the stage
  return sizeof(float) * ((size_t)ns * k.stage_floats + (size_t)2 * kMaxWaves * 256 +
                          (size_t)2 * pt * kMaxWaves * 256 + kt);
}

size_t fold_lds_bytes(const M3K& k, int ns) {
  const int WN = k.dqk / 16;
  return sizeof(float) * ((size_t)ns * k.stage_floats + (size_t)WN * 16 * kKtStride);
}

// Blocks of the fold kernel kf launches that one CU holds at once with `lds` bytes of LDS
// each: its registers limit them as well as its LDS (the rank-4 MIMO fold's 88 VGPRs
// allow five waves a SIMD, so two blocks of eight waves a CU where LDS would allow three).
template <int R, bool MIMO>
int fold_resident(const M3K& kf, size_t lds, bool narrow) {
  int n = 0;
  auto occ = [&](const void* kernel) {
    if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, kernel, 64 * (kf.dqk / 16), lds) !=
        hipSuccess) {
      (void)hipGetLastError();
      n = 1;
    }
  };
  const int pt = kf.ptiles;
  if (narrow) {
    if (pt == 4) occ(reinterpret_cast<const void*>(&m3_fold_kernel<R, MIMO, false, 4, kNarrowDma>));
    else if (pt == 2) occ(reinterpret_cast<const void*>(&m3_fold_kernel<R, MIMO, false, 2, kNarrowDma>));
    else occ(reinterpret_cast<const void*>(&m3_fold_kernel<R, MIMO, false, 1, kNarrowDma>));
  } else {
    if (pt == 4) occ(reinterpret_cast<const void*>(&m3_fold_kernel<R, MIMO, false, 4, kMaxDma>));
    else if (pt == 2) occ(reinterpret_cast<const void*>(&m3_fold_kernel<R, MIMO, false, 2, kMaxDma>));
    else occ(reinterpret_cast<const void*>(&m3_fold_kernel<R, MIMO, false, 1, kMaxDma>));
  }
  return n;
}

int fold_resident_any(const M3K& kf, size_t lds, bool narrow) {
  if (kf.psi == nullptr) return fold_resident<1, false>(kf, lds, narrow);
  const int R = 16 / kf.steps_per_chunk;
  if (R == 1) return fold_resident<1, true>(kf, lds, narrow);
  if (R == 2) return fold_resident<2, true>(kf, lds, narrow);
  return fold_resident<4, true>(kf, lds, narrow);
}

template <int R, bool MIMO, int PT, int MD>
hipError_t launch_fold(const M3K& kf, bool rev, hipStream_t st) {
  const long long blocks = (long long)kf.seg_blocks * kf.nsub;
  const size_t lds = fold_lds_bytes(kf, kf.nstages);
  const dim3 grid((unsigned)blocks), wg(64 * (kf.dqk / 16));
  if (rev) hipLaunchKernelGGL((m3_fold_kernel<R, MIMO, true, PT, MD>), grid, wg, lds, st, kf);
  else hipLaunchKernelGGL((m3_fold_kernel<R, MIMO, false, PT, MD>), grid, wg, lds, st, kf);
  return hipGetLastError();
}

template <int R, bool MIMO, int PT, bool ZOWN, int MD>
hipError_t launch_chunk(const M3K& k, bool rev, hipStream_t st) {
  const int WN = k.dqk / 16;
  const long long blocks = 8LL * (k.nparts / PT) * ((k.nseq + 7) / 8) * (k.split ? 2 : 1);
  const size_t lds = chunk_lds_bytes(k, PT, k.nstages);
  if (k.ang) {  // forward only: theta is a forward cumsum
    if (rev) return hipErrorInvalidValue;
    hipLaunchKernelGGL((m3_chunk_kernel<R, MIMO, false, PT, true, false, ZOWN, MD>),
                       dim3((unsigned)blocks), dim3(64 * (WN + 2 * PT)), lds, st, k);
  } else if (k.accum) {
    if constexpr (R == 1 && !MIMO) {
      if (rev)
        hipLaunchKernelGGL((m3_chunk_kernel<1, false, true, PT, false, true, ZOWN, MD>),
                           dim3((unsigned)blocks), dim3(64 * (WN + 2 * PT)), lds, st, k);
      else
        hipLaunchKernelGGL((m3_chunk_kernel<1, false, false, PT, false, true, ZOWN, MD>),
                           dim3((unsigned)blocks), dim3(64 * (WN + 2 * PT)), lds, st, k);
    } else {
      return hipErrorInvalidValue;  // accumulation is SISO only (m3_scan checks it)
    }
  } else if (rev) {
    hipLaunchKernelGGL((m3_chunk_kernel<R, MIMO, true, PT, false, false, ZOWN, MD>),
                       dim3((unsigned)blocks), dim3(64 * (WN + 2 * PT)), lds, st, k);
  } else {
    hipLaunchKernelGGL((m3_chunk_kernel<R, MIMO, false, PT, false, false, ZOWN, MD>),
                       dim3((unsigned)blocks), dim3(64 * (WN + 2 * PT)), lds, st, k);
  }
  return hipGetLastError();
}

// The scan, preceded when its sequences are split (k.split) by the fold of their head
// segments (kf: the same problem, its stage without z), on the same DMA plan width.
template <int R, bool MIMO>
hipError_t launch_chunk_pt(const M3K& k, const M3K& kf, bool rev, hipStream_t st) {
  const bool narrow = k.n_ins <= kNarrowDma * (k.dqk / 16);
  auto go = [&](auto zown, auto md) {
    constexpr bool Z = decltype(zown)::value;
    constexpr int M = decltype(md)::value;
    if (k.split) {
      const hipError_t e = kf.ptiles == 4   ? launch_fold<R, MIMO, 4, M>(kf, rev, st)
                           : kf.ptiles == 2 ? launch_fold<R, MIMO, 2, M>(kf, rev, st)
                                            : launch_fold<R, MIMO, 1, M>(kf, rev, st);
      if (e != hipSuccess) return e;
    }
    return k.ptiles == 2 ? launch_chunk<R, MIMO, 2, Z, M>(k, rev, st)
                         : launch_chunk<R, MIMO, 1, Z, M>(k, rev, st);
  };
  using T = std::true_type;
  using F = std::false_type;
  using Nd = std::integral_constant<int, kNarrowDma>;
  using Wd = std::integral_constant<int, kMaxDma>;
  if (k.zown) return narrow ? go(T{}, Nd{}) : go(T{}, Wd{});
  return narrow ? go(F{}, Nd{}) : go(F{}, Wd{});
}

}  // namespace

bool m3_chunk_supported(const M3Problem& pr) {
  const bool mimo = pr.psi != nullptr;
  const bool rank_ok = mimo ? (pr.rank == 1 || pr.rank == 2 || pr.rank == 4) : pr.rank == 1;
  // 32-bit offsets within a sequence: q/k, cos/sin and v/z/out spans below 2^30 floats
  const size_t lim = (size_t)1 << 30;
  const long long llim = (long long)lim;
  auto step_ok = [&](long long s) { return s >= 0 && s < llim && s * (long long)pr.len < llim; };
  const bool spans = pr.len * pr.rank * pr.groups * pr.dqk < lim &&
                     pr.len * pr.heads * pr.dv < lim && pr.len * pr.heads * pr.dqk < lim &&
                     step_ok(pr.v_strides[1]) && step_ok(pr.z_strides[1]) &&
                     step_ok(pr.ang_strides[1]);
  return rank_ok && pr.dv % 16 == 0 && pr.dqk % 16 == 0 && pr.dqk >= 16 &&
         pr.dqk <= 16 * (size_t)kMaxWaves && pr.len > 0 && spans;
}

hipError_t m3_scan_chunked(const M3Problem& pr, hipStream_t st) {
  M3K k{};
  k.q = pr.q; k.k = pr.k; k.v = pr.v; k.adt = pr.adt; k.dt = pr.dt; k.trap = pr.trap;
  k.qb = pr.q_bias; k.kb = pr.k_bias; k.cos = pr.cos; k.sin = pr.sin; k.D = pr.D; k.z = pr.z;
  k.psi = pr.psi; k.zeta = pr.zeta; k.phi = pr.phi;
  k.out = pr.out; k.last_state = pr.last_state; k.last_bx = pr.last_bx;
  k.out_tm = pr.out_time_major;
  k.accum = pr.accumulate;
  k.heads = (int)pr.heads; k.dv = (int)pr.dv; k.dqk = (int)pr.dqk;
  k.len = (int)pr.len; k.groups = (int)pr.groups;
  const int R = (int)pr.rank;
  k.nparts = k.dv / 16;
  k.steps_per_chunk = 16 / R;
  k.nchunks = (k.len + k.steps_per_chunk - 1) / k.steps_per_chunk;
  k.nseq = (int)(pr.batch * pr.heads);
  const int WN = k.dqk / 16;
  // Two dv slices per block share the q/k/cos/sin rows and G when dv allows.
  k.ptiles = (k.nparts % 2 == 0 && WN >= 2) ? 2 : 1;
  k.ang = pr.angles;
  k.nang = (int)pr.n_angles;
  k.vb = pr.v_strides[0]; k.vt = (int)pr.v_strides[1];
  k.zb = pr.z_strides[0]; k.zt = (int)pr.z_strides[1];
  k.zown = pr.z != nullptr && k.zt != k.vt;
  k.ab = pr.ang_strides[0]; k.at = (int)pr.ang_strides[1]; k.ah = pr.ang_strides[2];
  k.rec_floats = rec_floats((int)pr.rank, pr.angles != nullptr);
  auto plan = [&]() {
    const int T = k.steps_per_chunk;
    k.n_cs = pr.angles ? 0 : (T * (k.dqk / 8) + 63) / 64;
    k.n_ang = pr.angles ? (T * (k.nang / 4) + 63) / 64 : 0;
    k.n_v = (T * 4 * k.ptiles + 63) / 64;
    k.n_z = pr.z ? k.n_v : 0;
    k.n_ins = 2 * WN + 2 * k.n_cs + k.n_ang + k.n_v + k.n_z + (k.rec_floats / 4 + 63) / 64;
    k.stage_floats = k.n_ins * 256;
  };
  plan();
  k.nstages = kStages;
  while (k.nstages > 2 && chunk_lds_bytes(k, k.ptiles, k.nstages) > kLdsBudget) --k.nstages;
  if (chunk_lds_bytes(k, k.ptiles, k.nstages) > kLdsBudget && k.ptiles > 1) {
    k.ptiles = 1;
    plan();
  }
  if (chunk_lds_bytes(k, k.ptiles, k.nstages) > kLdsBudget) return hipErrorInvalidValue;
  if (k.n_ins > kMaxDma * WN) return hipErrorInvalidValue;  // DMA by the WN partial waves

  // Too few sequences for the chip. A block takes a whole CU (its LDS), so with P
  // blocks on C > P CUs, C - P CUs idle through the scan. Each sequence is then cut at
  // chunk `split`: a fold pass first computes the state every sequence reaches there
  // (the state update alone), then the scan runs 2P blocks, the P that resume at
  // `split` first and the P head segments [0, split) after them, several in turn on
  // the CUs the first P leave free. With deep = ceil(P / (C - P)) head segments per
  // free CU, each paying its ring's fill and drain (about 2 NS chunks), split =
  // (nchunks - 2 NS (deep - 1)) / (deep + 1) ends both groups together (configs 3 and
  // 4: 192 blocks on 256 CUs, deep 3, split near a quarter). The fold costs about 0.7
  // of a scan chunk per chunk at rank 1 and 0.4 at rank 4 (rank-4 chunks hold 4 steps
  // whose state update is a quarter of their work), so rank 1 splits from 256 chunks
  // (measured at B4 H24 against whole sequences: L 2048 +5%, 4096 -2%, 8192 -7%) and
  // other ranks from 64 (rank 4: L 1024 -5%, 2048 -11%, 4096 -14%, 8192 -16%). With the
  // fused angle pre-pass (SISO) the fold pieces rotate by theta from their own start and
  // the resuming blocks rotate each piece's state by theta at the piece's start (the
  // pieces' increments summed); MIMO keeps whole sequences.
  M3K kf = k;
  const long long blocks = (long long)k.nseq * (k.nparts / k.ptiles);
  const int cus = device_cus();
  const int min_chunks = R == 1 ? kMinSplitChunksRank1 : kMinSplitChunks;
  if ((!pr.angles || !k.psi) && cus > 0 && blocks < cus && k.nchunks >= min_chunks &&
      2 * chunk_lds_bytes(k, k.ptiles, k.nstages) > kLdsBudget) {
    const long long deep = (blocks + (cus - blocks) - 1) / (cus - blocks);
    const int split =
        (int)((k.nchunks - 2LL * k.nstages * (deep - 1)) / (deep + 1));
    if (split >= kMinSplitChunks / 4 && split < k.len / k.steps_per_chunk) {
      k.split = split;
      k.seg_blocks = 8 * (k.nparts / k.ptiles) * ((k.nseq + 7) / 8);
      kf.split = split;
      kf.z = nullptr;  // the fold's stage: the scan's without q and z
      kf.zown = 0;
      kf.n_z = 0;
      kf.skip_q = 1;
      // a fold block takes up to four dv slices (the scan two), so that the k, cos and
      // sin rows it shares across slices are fetched once for four (configs 3 and 4)
      const int T = k.steps_per_chunk;
      auto fold_plan = [&](int pt) {
        kf.ptiles = pt;
        kf.n_v = (T * 4 * pt + 63) / 64;
        kf.n_ins = WN + 2 * k.n_cs + k.n_ang + kf.n_v + (k.rec_floats / 4 + 63) / 64;
        kf.stage_floats = kf.n_ins * 256;
      };
      const int wide = k.n_ins <= kNarrowDma * WN ? kNarrowDma : kMaxDma;  // the scan's plan
      fold_plan(k.nparts % 4 == 0 ? 4 : k.ptiles);
      if (kf.n_ins > wide * WN) fold_plan(k.ptiles);
      const long long fblocks = (long long)k.nseq * (k.nparts / kf.ptiles);
      // up to three fold blocks per CU, as many as the CU holds with a ring of two stages
      // (a shallow ring each: latency is covered by the other blocks' waves; LDS and
      // registers both limit them), and the head segment in as many pieces as keep every
      // fold block resident at once: a second round of blocks would double the pass
      // (config 3: two blocks per CU, five pieces of 12 chunks, 480 blocks; eight pieces,
      // 768 blocks, ran in two rounds)
      const bool narrow = k.n_ins <= kNarrowDma * WN;  // the DMA plan launch_chunk_pt takes
      int bpc = 3;
      while (bpc > 1 && (bpc * fold_lds_bytes(kf, 2) > kLdsBudget ||
                         fold_resident_any(kf, fold_lds_bytes(kf, 2), narrow) < bpc))
        --bpc;
      kf.nstages = kFoldStages;
      while (kf.nstages > 2 && bpc * fold_lds_bytes(kf, kf.nstages) > kLdsBudget) --kf.nstages;
      int nsub = (int)(bpc * (long long)cus / fblocks);
      nsub = nsub < 1 ? 1 : nsub > split ? split : nsub;
      k.sub_len = kf.sub_len = (split + nsub - 1) / nsub;
      k.nsub = kf.nsub = (split + k.sub_len - 1) / k.sub_len;
      kf.seg_blocks = 8 * (k.nparts / kf.ptiles) * ((k.nseq + 7) / 8);
    }
  }

  const size_t nrec = (size_t)k.nseq * k.nchunks;
  hipError_t e = stream_alloc((void**)&k.rec, nrec * k.rec_floats * sizeof(float), st);
  if (e != hipSuccess) return e;
  kf.rec = k.rec;
  if (k.split) {
    const size_t fs = (size_t)k.nsub * k.nseq * k.dv * k.dqk;
    const size_t ds = (size_t)k.nsub * k.nseq, ts = k.ang ? ds * 64 : 0;
    e = stream_alloc((void**)&k.fold, (fs + ds + ts) * sizeof(float), st);
    if (e != hipSuccess) {
      (void)hipFreeAsync(k.rec, st);
      return e;
    }
    k.fold_decay = k.fold + fs;
    k.theta = k.ang ? k.fold_decay + ds : nullptr;
    kf.fold = k.fold;
    kf.fold_decay = k.fold_decay;
    kf.theta = k.theta;
  }
  const unsigned gblocks = (unsigned)((nrec + 16 * R - 1) / (16 * R));  // 16R records a block
  const int rev = pr.reverse ? 1 : 0;
  if (R == 1) hipLaunchKernelGGL(m3_gates_kernel<1>, dim3(gblocks), dim3(256), 0, st, k, rev);
  else if (R == 2) hipLaunchKernelGGL(m3_gates_kernel<2>, dim3(gblocks), dim3(256), 0, st, k, rev);
  else hipLaunchKernelGGL(m3_gates_kernel<4>, dim3(gblocks), dim3(256), 0, st, k, rev);
  e = hipGetLastError();
  if (e == hipSuccess) {
    const bool mimo = pr.psi != nullptr;
    if (!mimo) e = launch_chunk_pt<1, false>(k, kf, rev, st);
    else if (R == 1) e = launch_chunk_pt<1, true>(k, kf, rev, st);
    else if (R == 2) e = launch_chunk_pt<2, true>(k, kf, rev, st);
    else e = launch_chunk_pt<4, true>(k, kf, rev, st);
  }
  hipError_t fe = hipFreeAsync(k.rec, st);
  if (k.fold) {
    const hipError_t fe2 = hipFreeAsync(k.fold, st);
    if (fe == hipSuccess) fe = fe2;
  }
  return e != hipSuccess ? e : fe;
}

}  // namespace armscan
