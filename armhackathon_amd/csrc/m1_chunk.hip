// Mamba-1 selective scan, one direction (forward or reverse index mode), on gfx950.
//
// Semantics: the reference's scalar::scan (kernel/arm-scan-core/src/scalar.rs:11-89),
// per (batch, channel) row and state n:
//   dt = softplus(delta + bias) (when asked);  h_n <- exp(dt A_n) h_n + dt u B_n
//   y = sum_n C_n h_n ;  out = (y + D u) silu(z) ;  last_state = h after the last step
// with reverse walking t = L-1 .. 0 while out[t] stays at index t.
//
// Decomposition. A row is cut into chunks of CH = LPR * I consecutive steps (in
// traversal order); one row is owned by LPR lanes of a wave (64 / LPR rows per
// wave), and lane j of the row owns steps [j*I, j*I + I) of the current chunk.
// The wave walks the chunks of its rows in order, carrying the per-state row
// state from chunk to chunk in LDS (wave-private, no barriers). Per chunk and
// state n:
//   pass 1  every lane discretises its I steps, a_i = 2^(dt_i * A_n log2 e),
//           b_i = dt_i u_i B_n,i, and folds them into one affine map (a_tot, b_tot),
//           with a_tot = 2^(A_n log2 e * sum dt) (one exp, not a product of I);
//           the row's first lane folds the carried state in;
//   scan    an inclusive DPP scan of the affine maps across the row's lanes
//           (Hillis-Steele, row_shr 1/2/4/8 and, for 64-lane rows, the two row
//           broadcasts) gives every lane the absolute state at the end of its
//           block; a row_shr/wave_shr by one turns that into each lane's entry state;
//   pass 2  each lane replays its steps from the entry state with the stored
//           (a_i, b_i), accumulating y_i += C_n,i h_i.
// exp(dt A) is evaluated exactly once per (step, state). B and C rows (shared by
// all channels of a batch/group) are read straight from memory through the
// caches with 16-byte loads, one state ahead of their use.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <type_traits>
#include <utility>

#include "scan_common.h"
#include "scan_launch.h"

namespace armscan {

namespace {

struct M1Kern {
  const float *u, *delta, *A, *B, *C, *D, *z, *bias, *h0;
  float *out, *last;
  long long L;
  int rows, dim, N, groups, group_size, softplus;
  // strided z/out (m1_tile_kernel<.., true>): element strides per batch, channel and
  // step, and the bytes of one batch's slab (every offset inside it fits 32 bits)
  long long zs_b, zs_d, zs_t, os_b, os_d, os_t;
  unsigned z_bytes, o_bytes;
  // strided u (m1_tile_kernel<.., SIO != 0>): per-lane buffer loads, as z's in SIO 1
  long long us_b, us_d, us_t;
  unsigned u_bytes;
  int u_strided;
  int z_dma;  // strided z and out staged through LDS (m1_tile_kernel<.., 2>)
  int u_dma;  // with z_dma: strided u (unit channel stride) through the same stage
  // Rows cut into `segs` segments of `seg_chunks` chunks when there are too few rows
  // to fill the chip: segmap[row][s][n] = (A, B), the affine map of segment s < segs-1
  // (h_end = A h_start + B), from m1_seg_fold_kernel. segs <= 1: whole rows.
  int segs;
  long long seg_chunks;
  float* segmap;
  // Row pitch of B and C in floats: L, or L rounded up to 4 when the tiled kernel reads
  // padded copies of rows that are not 16-byte multiples. bpo: zeros in front of each
  // padded row (ldb - L for reverse, whose chunks end at L, so that every chunk starts
  // on a 16-byte piece; 0 otherwise). B and C point at the rows' first data float.
  long long ldb, bpo;
};

// One traversal of a multi-traversal launch: its own inputs, B/C, outputs and
// direction (u/delta/z rows in traversal order up to the direction).
struct M1Job {
  const float *u, *delta, *z, *B, *C;
  float *out, *last;
  int rev;
};
constexpr int kMaxJobs = 4;
struct M1Jobs {
  M1Job job[kMaxJobs];
  int njobs, blocks_per_job;
};

constexpr int kWavesPerBlock = 4;
#ifndef M1_TILE_I
#define M1_TILE_I 16
#endif

// Inclusive Hillis-Steele scan steps as single VOP2 DPP instructions:
//   v_fmac_f32_dpp b, b[src], a   ->  b = a * b[src] + b
//   v_mul_f32_dpp  a, a[src], a   ->  a = a * a[src]
// Lanes without a source lane (row/wave edge, masked rows) are not written, so
// they keep their map (the identity step). Each DPP read of a VGPR needs two
// wait states after the VALU write of that VGPR; the s_nops provide them.
#define ARMSCAN_DPP_STEP(CTRL, MASK)                                           \
  "s_nop 0\n\t"                                                               \
  "v_fmac_f32_dpp %0, %0, %1 " CTRL " row_mask:" MASK " bank_mask:0xf\n\t"    \
  "s_nop 0\n\t"                                                               \
  "v_mul_f32_dpp %1, %1, %1 " CTRL " row_mask:" MASK " bank_mask:0xf\n\t"
#define ARMSCAN_DPP_LAST(CTRL, MASK) \
  "s_nop 0\n\t"                      \
  "v_fmac_f32_dpp %0, %0, %1 " CTRL " row_mask:" MASK " bank_mask:0xf\n\t"

// Scan primitives over one row of LPR lanes.
template <int LPR> struct Row;

template <> struct Row<16> {
  // inclusive scan of affine maps (a, b) over the 16 lanes of each DPP row;
  // on return b is the inclusive composition (a is left partially combined).
  static __device__ __forceinline__ void scan(float& a, float& b) {
    asm volatile("s_nop 1\n\t"
                 ARMSCAN_DPP_STEP("row_shr:1", "0xf")
                 ARMSCAN_DPP_STEP("row_shr:2", "0xf")
                 ARMSCAN_DPP_STEP("row_shr:4", "0xf")
                 ARMSCAN_DPP_LAST("row_shr:8", "0xf")
                 "s_nop 1"
                 : "+v"(b), "+v"(a));
  }
  // value of the previous lane of the row; the row's first lane gets `first`
  static __device__ __forceinline__ float prev(float v, float first) {
    return dpp<kRowShr1, 0xF>(first, v);
  }
  // the row's last lane's value, delivered to the row's first lane
  static __device__ __forceinline__ float last_to_first(float v) {
    return dpp<kRowMirror, 0xF>(0.0f, v);
  }
  // h = a0 * (b_incl of the previous lane) + h; the row's first lane keeps h
  static __device__ __forceinline__ void step_from_prev(float& h, float b_incl, float a0) {
    asm volatile("v_fmac_f32_dpp %0, %1, %2 row_shr:1 row_mask:0xf bank_mask:0xf"
                 : "+v"(h) : "v"(b_incl), "v"(a0));
  }
};

template <> struct Row<64> {
  static __device__ __forceinline__ void scan(float& a, float& b) {
    asm volatile("s_nop 1\n\t"
                 ARMSCAN_DPP_STEP("row_shr:1", "0xf")
                 ARMSCAN_DPP_STEP("row_shr:2", "0xf")
                 ARMSCAN_DPP_STEP("row_shr:4", "0xf")
                 ARMSCAN_DPP_STEP("row_shr:8", "0xf")
                 ARMSCAN_DPP_STEP("row_bcast:15", "0xa")
                 ARMSCAN_DPP_LAST("row_bcast:31", "0xc")
                 "s_nop 1"
                 : "+v"(b), "+v"(a));
  }
  static __device__ __forceinline__ float prev(float v, float first) {
    return dpp<kWaveShr1, 0xF>(first, v);
  }
  static __device__ __forceinline__ float last_to_first(float v) {
    return dpp<kWaveRor1, 0xF>(0.0f, v);
  }
  static __device__ __forceinline__ void step_from_prev(float& h, float b_incl, float a0) {
    asm volatile("v_fmac_f32_dpp %0, %1, %2 wave_shr:1 row_mask:0xf bank_mask:0xf"
                 : "+v"(h) : "v"(b_incl), "v"(a0));
  }
};

// Load the I steps of one lane block in traversal order: step i of the block
// starting at traversal index sb is memory t = sb + i (forward) or L-1-sb-i
// (reverse). Steps past the row's end read `fill`.
// Lv bounds the valid traversal indices (s < Lv); L is the row length used for
// the reverse mapping (a FULL chunk passes Lv = sb + I so the check folds away).
template <int I, bool REV, bool VEC>
__device__ __forceinline__ void load_block(const float* __restrict__ row, long long Lv,
                                           long long sb, float fill, float (&v)[I],
                                           long long L, long long ts = 1) {
  if (VEC) {
    const long long mb = REV ? L - sb - I : sb;
    const float4* p = reinterpret_cast<const float4*>(row + mb);
#pragma unroll
    for (int q = 0; q < I / 4; ++q) {
      const float4 x = p[q];
      const float w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) v[REV ? I - 1 - (4 * q + e) : 4 * q + e] = w[e];
    }
  } else {
#pragma unroll
    for (int i = 0; i < I; ++i) {
      const long long s = sb + i;
      v[i] = s < Lv ? row[(REV ? L - 1 - s : s) * ts] : fill;
    }
  }
}

template <int I, bool REV, bool VEC>
__device__ __forceinline__ void store_block(float* __restrict__ row, long long Lv, long long sb,
                                            const float (&v)[I], long long L, long long ts = 1) {
  if (VEC) {
    const long long mb = REV ? L - sb - I : sb;
    float4* p = reinterpret_cast<float4*>(row + mb);
#pragma unroll
    for (int q = 0; q < I / 4; ++q) {
      float w[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) w[e] = v[REV ? I - 1 - (4 * q + e) : 4 * q + e];
      p[q] = make_float4(w[0], w[1], w[2], w[3]);
    }
  } else {
#pragma unroll
    for (int i = 0; i < I; ++i) {
      const long long s = sb + i;
      if (s < Lv) row[(REV ? L - 1 - s : s) * ts] = v[i];
    }
  }
}

// Buffer resource over one batch's slab of a strided tensor (raw, unswizzled;
// reads past `bytes` return 0).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t slab_rsrc(const float* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(base), (short)0, (int)bytes,
                                           0x00020000);
}

// The I steps of a lane block of a strided row (steps `ts` floats apart, e.g. a
// (batch, dim, len) view of time-major storage): one VGPR offset, the block's
// lowest memory step, and a wave-uniform SGPR offset per step, so the addressing
// costs no VALU work.
template <int I, bool REV>
__device__ __forceinline__ void load_block_strided(__amdgpu_buffer_rsrc_t r, unsigned voff,
                                                   long long ts, float (&v)[I]) {
#pragma unroll
  for (int k = 0; k < I; ++k)
    v[REV ? I - 1 - k : k] = __builtin_bit_cast(
        float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, (int)(k * ts * 4), 0));
}

template <int I, bool REV>
__device__ __forceinline__ void store_block_strided(__amdgpu_buffer_rsrc_t r, unsigned voff,
                                                    long long ts, const float (&v)[I]) {
#pragma unroll
  for (int k = 0; k < I; ++k)
    __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v[REV ? I - 1 - k : k]),
                                          r, voff, (int)(k * ts * 4), 0);
}

// A lane block of the row's tail chunk in a strided row (steps `ts` floats apart):
// one base pointer at traversal step sb and wave-uniform offsets; steps past the
// row's end read 0 / are not written.
template <int I, bool REV>
__device__ __forceinline__ void load_tail(const float* row, long long L, long long sb,
                                          long long ts, float (&v)[I]) {
  const float* base = row + (REV ? L - 1 - sb : sb) * ts;
  const long long st = REV ? -ts : ts;
#pragma unroll
  for (int i = 0; i < I; ++i) v[i] = sb + i < L ? base[i * st] : 0.0f;
}

template <int I, bool REV>
__device__ __forceinline__ void store_tail(float* row, long long L, long long sb, long long ts,
                                           const float (&v)[I]) {
  float* base = row + (REV ? L - 1 - sb : sb) * ts;
  const long long st = REV ? -ts : ts;
#pragma unroll
  for (int i = 0; i < I; ++i)
    if (sb + i < L) base[i * st] = v[i];
}

// One state n of one chunk given this lane's B/C blocks (bb, cc): pass 1, the
// row scan, pass 2, and the carry into the next chunk. a2 = A[d][n] log2(e).
template <int LPR, int I>
__device__ __forceinline__ void state_core(int n, int j, float a2, float* carry,
                                           float* last_n, const float (&dt)[I],
                                           const float (&du)[I], float sdt, float (&y)[I],
                                           const float (&bb)[I], const float (&cc)[I]) {
  float a[I], b[I];
  float bt = 0.0f;
#pragma unroll
  for (int i = 0; i < I; ++i) {
    a[i] = ex2(dt[i] * a2);
    b[i] = du[i] * bb[i];
    bt = fmaf(a[i], bt, b[i]);
  }
  float at = ex2(a2 * sdt);
  const float hc_row = carry[n];
  const float hc = (j == 0) ? hc_row : 0.0f;
  bt = fmaf(at, hc, bt);  // the row's first lane starts from the carried state
  Row<LPR>::scan(at, bt);
  float h = Row<LPR>::prev(bt, hc);  // state entering this lane's block
#pragma unroll
  for (int i = 0; i < I; ++i) {
    h = fmaf(a[i], h, b[i]);
    y[i] = fmaf(cc[i], h, y[i]);
  }
  const float hend = Row<LPR>::last_to_first(h);
  if (j == 0) carry[n] = hend;
  if (last_n && j == LPR - 1) *last_n = h;
}

// One state of the global-load path: the next state's B/C blocks are fetched
// into (b1, c1) while this one computes from (b0, c0).
template <int LPR, int I, bool REV, bool V>
__device__ __forceinline__ void state(const M1Kern& p, int n, long long sb, long long Lv, int j,
                                      bool valid, bool last_chunk, long long row,
                                      const float* Bg, const float* Cg, const float* a2s,
                                      float* carry, const float (&dt)[I], const float (&du)[I],
                                      float sdt, float (&y)[I], const float (&b0)[I],
                                      const float (&c0)[I], float (&b1)[I], float (&c1)[I]) {
  const long long L = p.L;
  if (n + 1 < p.N) {
    load_block<I, REV, V>(Bg + (long long)(n + 1) * L, Lv, sb, 0.0f, b1, L);
    load_block<I, REV, V>(Cg + (long long)(n + 1) * L, Lv, sb, 0.0f, c1, L);
  }
  float* last_n = (last_chunk && p.last && valid) ? p.last + row * p.N + n : nullptr;
  state_core<LPR, I>(n, j, a2s[n], carry, last_n, dt, du, sdt, y, b0, c0);
}

// One chunk of a wave's rows. FULL: every lane's block lies inside the row
// (no bounds checks; 16-byte accesses when VEC); otherwise the row's tail.
// (dn, un) carry the raw delta/u blocks of this chunk when `have` (fetched during
// the previous chunk); when `pre_sb` >= 0 this chunk fetches the next chunk's
// blocks (at traversal base pre_sb) into them half-way through its states.
template <int LPR, int I, bool REV, bool VEC, bool FULL>
__device__ __forceinline__ void chunk(const M1Kern& p, long long sb, int j, bool valid,
                                      bool last_chunk, long long row, const float* urow,
                                      const float* drow, const float* zrow, float* orow,
                                      const float* Bg, const float* Cg, const float* a2s,
                                      float bias, float dskip, float* carry, float (&dn)[I],
                                      float (&un)[I], bool have, long long pre_sb,
                                      long long zts = 1, long long ots = 1,
                                      long long uts = 1) {
  constexpr bool V = VEC && FULL;
  const long long L = p.L;
  const int N = p.N;
  const long long Lv = FULL ? sb + I : L;  // FULL: the block is known to fit
  float dt[I], du[I], y[I];
  float sdt = 0.0f;
  if (!have) {
    load_block<I, REV, V>(drow, Lv, sb, 0.0f, dn, L);
    load_block<I, REV, V>(urow, Lv, sb, 0.0f, un, L, uts);  // uts != 1 only with !V
  }
#pragma unroll
  for (int i = 0; i < I; ++i) {
    float x = dn[i] + bias;
    if (p.softplus) x = softplus_fast(x);
    if (!FULL) x = (sb + i < L) ? x : 0.0f;  // padding steps are the identity map
    dt[i] = x;
    du[i] = x * un[i];
    y[i] = dskip * un[i];
    sdt += x;
  }
  if (!FULL) {
    // the row's tail: bounds-checked loads, no prefetching (keeps registers low)
    for (int n = 0; n < N; ++n) {
      float bb[I], cc[I];
      load_block<I, REV, false>(Bg + (long long)n * L, Lv, sb, 0.0f, bb, L);
      load_block<I, REV, false>(Cg + (long long)n * L, Lv, sb, 0.0f, cc, L);
      float* last_n = (last_chunk && p.last && valid) ? p.last + row * N + n : nullptr;
      state_core<LPR, I>(n, j, a2s[n], carry, last_n, dt, du, sdt, y, bb, cc);
    }
    if (zrow) {
      float zz[I];
      load_block<I, REV, false>(zrow, Lv, sb, 0.0f, zz, L, zts);
#pragma unroll
      for (int i = 0; i < I; ++i) y[i] *= silu_fast(zz[i]);
    }
    if (valid) store_block<I, REV, false>(orow, Lv, sb, y, L, ots);
    return;
  }
  float bv[I], cv[I], bn[I], cn[I], zz[I];
  load_block<I, REV, V>(Bg, Lv, sb, 0.0f, bv, L);
  load_block<I, REV, V>(Cg, Lv, sb, 0.0f, cv, L);
  const int half = (N / 2) & ~1;
  // states in pairs, ping-ponging the B/C registers: state n computes from
  // (bv, cv) while the loads of state n+1 land in (bn, cn)
  for (int n = 0; n < N; n += 2) {
    if (n == half && pre_sb >= 0) {
      load_block<I, REV, VEC>(drow, L, pre_sb, 0.0f, dn, L);
      load_block<I, REV, VEC>(urow, L, pre_sb, 0.0f, un, L);
    }
    if (zrow && n + 2 >= N) load_block<I, REV, V>(zrow, Lv, sb, 0.0f, zz, L);
    state<LPR, I, REV, V>(p, n, sb, Lv, j, valid, last_chunk, row, Bg, Cg, a2s, carry, dt, du,
                          sdt, y, bv, cv, bn, cn);
    if (n + 1 < N)
      state<LPR, I, REV, V>(p, n + 1, sb, Lv, j, valid, last_chunk, row, Bg, Cg, a2s, carry,
                            dt, du, sdt, y, bn, cn, bv, cv);
  }
  if (zrow) {
#pragma unroll
    for (int i = 0; i < I; ++i) y[i] *= silu_fast(zz[i]);
  }
  if (valid) store_block<I, REV, V>(orow, Lv, sb, y, L);
}

template <int LPR, int I, bool REV, bool VEC>
__global__ void __launch_bounds__(64 * kWavesPerBlock, 2)
m1_chunk_kernel(M1Kern p) {
  constexpr int RPW = 64 / LPR;  // rows per wave
  constexpr long long CH = (long long)LPR * I;
  extern __shared__ float s_lds[];  // carry [wave][row][N], then A*log2e [wave][row][N]

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = lane % LPR;
  const int rw = lane / LPR;
  const long long row_raw = ((long long)blockIdx.x * kWavesPerBlock + wave) * RPW + rw;
  const bool valid = row_raw < p.rows;
  const long long row = valid ? row_raw : (long long)p.rows - 1;
  const long long L = p.L;
  const int N = p.N;
  const int bi = (int)(row / p.dim), d = (int)(row - (long long)bi * p.dim);
  const int g = d / p.group_size;
  const float* urow = p.u + row * L;
  const float* drow = p.delta + row * L;
  const float* zrow = p.z ? p.z + row * L : nullptr;
  float* orow = p.out + row * L;
  const float* Bg = p.B + ((long long)bi * p.groups + g) * N * L;
  const float* Cg = p.C + ((long long)bi * p.groups + g) * N * L;
  const float* Arow = p.A + (long long)d * N;
  const float bias = p.bias ? p.bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;
  float* carry = s_lds + (wave * RPW + rw) * N;
  float* a2s = s_lds + (kWavesPerBlock * RPW + wave * RPW + rw) * N;

  if (j == 0)
    for (int n = 0; n < N; ++n) {
      carry[n] = p.h0 ? p.h0[row * N + n] : 0.0f;
      a2s[n] = Arow[n] * kLog2e;
    }

  const long long nch = (L + CH - 1) / CH;
  const long long nfull = L / CH;  // chunks that lie entirely inside the row
  float dn[I], un[I];
  for (long long c = 0; c < nfull; ++c) {
    const long long pre = c + 1 < nfull ? (c + 1) * CH + (long long)j * I : -1;
    chunk<LPR, I, REV, VEC, true>(p, c * CH + (long long)j * I, j, valid, c + 1 == nch, row,
                                  urow, drow, zrow, orow, Bg, Cg, a2s, bias, dskip, carry, dn,
                                  un, c > 0, pre);
  }
  if (nfull < nch)
    chunk<LPR, I, REV, VEC, false>(p, nfull * CH + (long long)j * I, j, valid, true, row, urow,
                                   drow, zrow, orow, Bg, Cg, a2s, bias, dskip, carry, dn, un,
                                   false, -1);
}

// ---------------------------------------------------------------------------
// LDS-tiled variant (16 lanes x I steps per row, 4 rows per wave, 16 rows per
// block, all in one batch/group). B and C are the per-element operands that
// dominate the on-chip traffic (two floats per step and state in every lane),
// so instead of each wave pulling them through the L1 the block stages them
// once per chunk in LDS, in tiles of kTileStates states x CH = 16*I steps (B
// rows then C rows), double-buffered and filled by direct-to-LDS DMA
// (global_load_lds_dwordx4): no VGPRs are spent on staging and the next tile
// streams in while the current one is consumed. One barrier per tile.
//
// Tile row layout: a row of CH floats is 4I pieces of 4 floats; lane j of a
// DPP row reads its I/4 pieces (j' = j forward, 15-j reverse) with I/4
// ds_read_b128, the q-th of which hits slot 16q + j' of the row: the 16 lanes of
// each read touch 256 contiguous bytes (no bank conflicts). Slot t of a row
// therefore holds piece (I/4)(t mod 16) + t/16, and that is what the DMA writes.
constexpr int kTileStates = 8;

template <int I> struct Tile {
  static constexpr int CH = 16 * I;                    // steps per chunk (row floats)
  static constexpr int QP = I / 4;                     // pieces per lane
  static constexpr int FLOATS = 2 * kTileStates * CH;  // B rows then C rows
  static constexpr int DMA = FLOATS / 256;             // wave-wide 16-byte DMA ops
};

template <int I, bool REV>
__device__ __forceinline__ void lds_block(const float* __restrict__ trow, int j,
                                          float (&v)[I]) {
  const int jj = REV ? 15 - j : j;
  const float4* t = reinterpret_cast<const float4*>(trow);
#pragma unroll
  for (int q = 0; q < I / 4; ++q) {
    const float4 x = t[16 * q + jj];
    const float w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) v[REV ? I - 1 - (4 * q + e) : 4 * q + e] = w[e];
  }
}

// DMA one tile (states n0 .. n0+kTileStates-1 of the chunk whose memory range
// starts at mem0) into `tile`. Each DMA op fills 256 consecutive tile floats with
// 16-byte pieces; the block's waves take turns. DW (rows of B/C not 16-byte aligned:
// L % 4 != 0 or an unaligned base) moves single floats instead, 64 to an op, into
// the same layout. `part`: the row's tail chunk, whose range runs past the row; the
// positions past it are read from kZeroPiece, so that they hold 0 as the general
// path's bounds-checked loads give.
__device__ __align__(16) float kZeroPiece[4] = {0.0f, 0.0f, 0.0f, 0.0f};

template <int I, bool DW = false>
__device__ __forceinline__ void issue_tile(float* tile, const float* Bg, const float* Cg,
                                           long long L, long long ldb, long long bpo,
                                           long long mem0, int n0, int N, int wave, int lane,
                                           bool part = false) {
  using G = Tile<I>;
  if constexpr (!DW) {
    constexpr int SPR = G::CH / 4;  // slots per tile row
    const int t = lane % SPR;
    const int piece = G::QP * (t & 15) + (t >> 4);
#pragma unroll
    for (int m0 = 0; m0 < G::DMA; m0 += kWavesPerBlock) {
      const int m = m0 + wave;  // wave-uniform
      if (G::DMA % kWavesPerBlock == 0 || m < G::DMA) {
        const int k = m * (256 / G::CH) + lane / SPR;  // tile row of this lane
        const int n = n0 + (k % kTileStates);
        if (n < N && (k < kTileStates || Cg != nullptr)) {  // Cg null: B rows only
          // a piece lies wholly inside the (padded) row [-bpo, ldb - bpo) or outside it
          const long long g = mem0 + 4 * piece;
          const float* src = part && (g < -bpo || g >= ldb - bpo)
                                 ? kZeroPiece
                                 : (k < kTileStates ? Bg : Cg) + (long long)n * ldb + g;
          __builtin_amdgcn_global_load_lds(
              (const void*)src, (__attribute__((address_space(3))) void*)(tile + m * 256), 16,
              0, 0);
        }
      }
    }
  } else {
    constexpr int OPS = G::FLOATS / 64;  // single-float ops per tile
    static_assert(OPS % kWavesPerBlock == 0, "whole rounds of ops per wave");
#pragma unroll
    for (int m0 = 0; m0 < OPS; m0 += kWavesPerBlock) {
      const int m = m0 + wave;  // wave-uniform
      const int f = m * 64 + lane;  // tile float of this lane
      const int k = f / G::CH, fr = f % G::CH;  // tile row, float in the row
      const int t = fr >> 2;                   // its 16-byte slot
      const int col = 4 * (G::QP * (t & 15) + (t >> 4)) + (fr & 3);
      const int n = n0 + (k % kTileStates);
      if (n < N && (k < kTileStates || Cg != nullptr)) {
        const long long g = mem0 + col;
        const float* src = part && (g < 0 || g >= L)
                               ? kZeroPiece
                               : (k < kTileStates ? Bg : Cg) + (long long)n * ldb + g;
        __builtin_amdgcn_global_load_lds(
            (const void*)src, (__attribute__((address_space(3))) void*)(tile + m * 64), 4, 0,
            0);
      }
    }
  }
}

// Strided z through LDS: the block's 16 channels of a chunk's 256 steps, as
// [step][channel] (16 KB). With zs_d == 1 the four channels 4q .. 4q+3 of a step
// are one 16-byte piece, so the block fetches whole 64-byte runs instead of each
// wave pulling 16 bytes out of every line it touches. DMA op m holds the steps
// 16m .. 16m+15 (lane block m of the chunk); its slot L holds piece
// x = L ^ m: step 16m + x/4, channels 4(x%4) .. +3 — the XOR spreads the 16 lanes
// that read one step of their blocks over the banks. `part`: the row's tail chunk,
// whose steps past the row's end are read from kZeroPiece (0, as the bounds-checked
// loads give).
constexpr int kZStageFloats = 16 * 256;

// The zero row after the carries, A*log2e and the tile state's inputs sits 8 floats past
// their end: a row's first lane reads its carry where the other 15 read the zero row, and
// both were on bank n (rows of 16 floats from a 32-float-aligned base), a two-way
// conflict on every state.
constexpr int kZerosPad = 8;

template <bool REV>
__device__ __forceinline__ void issue_z_stage(float* zbuf, const float* zslab, long long zs_t,
                                              long long L, long long c0, int d0, int wave,
                                              int lane, bool part = false) {
  // recomputed per chunk: hoisting these addresses out of the chunk loop would hold
  // registers through the whole scan
  asm volatile("" : "+v"(lane));
#pragma unroll
  for (int m0 = 0; m0 < 16; m0 += kWavesPerBlock) {
    const int m = m0 + wave;  // wave-uniform
    const int x = lane ^ m;
    const long long s = c0 + 16 * m + (x >> 2);  // traversal step
    const float* src = part && s >= L ? kZeroPiece
                                      : zslab + d0 + 4 * (x & 3) + (REV ? L - 1 - s : s) * zs_t;
    __builtin_amdgcn_global_load_lds((const void*)src,
                                     (__attribute__((address_space(3))) void*)(zbuf + m * 256),
                                     16, 0, 0);
  }
}

// Lane (row rw of wave w, lane block j): steps 16j + i of channel 4w + rw sit in
// slot (4i + w) ^ j of DMA op j, i.e. 4(i ^ (j>>2)) + (w ^ (j&3)).
__device__ __forceinline__ void read_z_stage(const float* zbuf, int j, int wave, int rw,
                                             float (&v)[16]) {
  asm volatile("" : "+v"(j));  // keep the addresses out of the chunk loop's registers
  const float* base = zbuf + j * 256 + 4 * (wave ^ (j & 3)) + rw;
  const int jh = j >> 2;
#pragma unroll
  for (int i = 0; i < 16; ++i) v[i] = base[16 * (i ^ jh)];
}

// The outputs through the same stage, the other way round: each lane writes its
// 16 steps of its channel into the swizzled layout above; after a sync, lane l of
// wave w stores slot l ^ m of op m = 4r + w (r = 0..3): step 16m + l/4, channels
// 4(l%4) .. +3, so four adjacent lanes store one step's 16 channels as 64 bytes.
// (Strided per-lane stores put the four channels of a step in lanes 16 apart, which
// the memory pipeline does not combine.)
__device__ __forceinline__ void write_out_stage(float* zbuf, int j, int wave, int rw,
                                                const float (&v)[16]) {
  asm volatile("" : "+v"(j));
  float* base = zbuf + j * 256 + 4 * (wave ^ (j & 3)) + rw;
  const int jh = j >> 2;
#pragma unroll
  for (int i = 0; i < 16; ++i) base[16 * (i ^ jh)] = v[i];
}

// `part`: the row's tail chunk, whose steps past the row's end are not stored.
template <bool REV>
__device__ __forceinline__ void store_out_stage(const float* zbuf, float* oslab, long long os_t,
                                                long long L, long long c0, int d0, int wave,
                                                int lane, bool part = false) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int m = 4 * r + wave;
    const float4 v = *reinterpret_cast<const float4*>(zbuf + m * 256 + 4 * (lane ^ m));
    const long long s = c0 + 16 * m + (lane >> 2);  // traversal step
    if (!part || s < L)
      *reinterpret_cast<float4*>(oslab + d0 + 4 * (lane & 3) + (REV ? L - 1 - s : s) * os_t) =
          v;
  }
}


// Issue priority of this wave from its progress through its tiles: 3 for the first
// half, 2 to three quarters, 1 to 90%, 0 after. The SIMD arbiter otherwise favours the
// oldest wave, so the three waves sharing a SIMD (one per resident block, dispatched
// one after another) finish in dispatch order and leave the SIMD to a single wave for
// the last fifth of the kernel (measured with per-wave s_memrealtime stamps: waves of
// the same work ending at 84, 114 and 136 us). A wave that is ahead now yields to the
// ones behind it; the headline scan runs about 5% faster.
// The share is compared without a division (floor(100 k / n) < t exactly when
// 100 k < t n): a 64-bit division per tile costs about 130 scalar instructions.
__device__ __forceinline__ void progress_prio(long long k, long long ntiles) {
  const long long k100 = 100 * k;
  if (k100 < 50 * ntiles) __builtin_amdgcn_s_setprio(3);
  else if (k100 < 75 * ntiles) __builtin_amdgcn_s_setprio(2);
  else if (k100 < 90 * ntiles) __builtin_amdgcn_s_setprio(1);
  else __builtin_amdgcn_s_setprio(0);
}

// Workgroup barrier that waits for LDS accesses only (global stores stay in flight).
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ void tile_sync() {
  __builtin_amdgcn_s_waitcnt(0);  // this wave's DMA (and every other access) landed
  __syncthreads();
}

// State core of the tiled path. hc is the carried row state in the row's first
// lane and 0 in the others; it is folded into b_0 so that pass 1's aggregate
// and pass 2's first step include it. The row's last lane returns the state at
// the end of the chunk (the value in other lanes is meaningless).
template <int I>
__device__ __forceinline__ float tile_state(float a2, float hc, const float (&dt)[I],
                                            const float (&du)[I], float sdt, float (&y)[I],
                                            const float (&bb)[I], const float (&cc)[I]) {
  float a[I], b[I];
#pragma unroll
  for (int i = 0; i < I; ++i) {
    a[i] = ex2(dt[i] * a2);
    b[i] = du[i] * bb[i];
  }
  b[0] = fmaf(a[0], hc, b[0]);
  float bt = b[0];
#pragma unroll
  for (int i = 1; i < I; ++i) bt = fmaf(a[i], bt, b[i]);
  float at = ex2(a2 * sdt);
  Row<16>::scan(at, bt);
  float h = b[0];
  Row<16>::step_from_prev(h, bt, a[0]);  // state after this lane's first step
  y[0] = fmaf(cc[0], h, y[0]);
#pragma unroll
  for (int i = 1; i < I; ++i) {
    h = fmaf(a[i], h, b[i]);
    y[i] = fmaf(cc[i], h, y[i]);
  }
  return h;
}

// The states n0 .. n0+kTileStates-1 of one chunk from one LDS tile, unrolled so
// that the LDS offsets are immediates. cbase points at the row's carries for
// the row's first lane and at zeros for the others.
template <int I, bool REV>
__device__ __forceinline__ void tile_states(const float* tile, int n0, int N, int j,
                                            const float* a2s, const float* cbase,
                                            float* carry, float* last_row,
                                            const float (&dt)[I], const float (&du)[I],
                                            float sdt, float (&y)[I]) {
  constexpr int CH = Tile<I>::CH;
#pragma unroll
  for (int s = 0; s < kTileStates; ++s) {
    if (n0 + s < N) {
      float cc[I], bb[I];
      lds_block<I, REV>(tile + s * CH, j, bb);
      lds_block<I, REV>(tile + (kTileStates + s) * CH, j, cc);
      const float a2 = a2s[n0 + s];
      const float hc = cbase[n0 + s];
      const float h = tile_state<I>(a2, hc, dt, du, sdt, y, bb, cc);
      if (j == 15) {
        carry[n0 + s] = h;
        if (last_row) last_row[n0 + s] = h;
      }
    }
  }
}

// The rows of block `blk` (16 per block) through one traversal. SIO 0: z and out
// (batch, dim, len) contiguous; 1: strided (p.zs_*, p.os_*), z read with buffer
// loads and out written with buffer stores; 2: strided with unit channel stride,
// z and out staged through LDS; 3: as 2, with u staged through the same LDS buffer
// (its own compile-time case, so that the per-lane u loads of 1 and 2 hold no
// registers in it). ALN: rows 16-byte aligned (L % 4 == 0, aligned bases), so that
// rows move in 16-byte pieces; otherwise single floats (SIO 0 only).
// The row's tail chunk (L % 256 steps) runs in the tile loop as well: its loads and
// stores check bounds (per lane, by strides, for SIO 1; in the DMA and the stores of
// the LDS stages of SIO 2 and 3), its B/C positions past the row read zeros, and its
// steps past the row's end are identity maps (dt = 0). TAIL: compiled only for rows with a tail chunk
// (L % 256 != 0), so that the kernels for whole chunks carry none of its code.
// DWBC: B/C rows are not 16-byte multiples in memory, and the tiles fill by single-float
// DMA (the allocation-free entry, the multi-traversal launch); otherwise their rows are
// (a padded copy of pitch p.ldb where L % 4 != 0).
template <int I, bool REV, int SIO, bool SEG = false, bool ALN = true, bool TAIL = false,
          bool DWBC = !ALN>
__device__ __forceinline__ void tile_rows(const M1Kern& p, long long blk, int seg = 0) {
  static_assert(ALN || SIO == 0, "unaligned rows: contiguous z and out only");
  constexpr int LPR = 16, RPW = 4;
  using G = Tile<I>;
  constexpr long long CH = G::CH;
  extern __shared__ __attribute__((aligned(16))) float s_lds[];
  float* tiles = s_lds;                                  // [2][G::FLOATS]
  float* zbuf = s_lds + 2 * G::FLOATS;  // SIO 2, 3: [256][16] z stage; !ALN: out stage
  float* small = zbuf + (SIO >= 2 || !ALN ? kZStageFloats : 0);  // carry, A*log2e, zeros

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = lane % LPR;
  const int rw = lane / LPR;
  const long long row = (blk * kWavesPerBlock + wave) * RPW + rw;
  const long long L = p.L;
  const int N = p.N;
  const int bi = (int)(row / p.dim), d = (int)(row - (long long)bi * p.dim);
  const int g = d / p.group_size;
  const bool ustr = SIO && p.u_strided;  // u read by strides (wave-uniform)
  const float* urow = ustr ? p.u + bi * p.us_b + d * p.us_d : p.u + row * L;
  const float* drow = p.delta + row * L;
  const float* zrow =
      p.z ? (SIO ? p.z + bi * p.zs_b + d * p.zs_d : p.z + row * L) : nullptr;
  float* orow = SIO ? p.out + bi * p.os_b + d * p.os_d : p.out + row * L;
  // strided z/out: the block's 16 rows share one batch, whose index taken from the
  // block id is wave-uniform (a buffer resource must be)
  const long long bib = blk * (kWavesPerBlock * RPW) / p.dim;
  const long long ldb = p.ldb;
  const float* Bg = p.B + ((long long)bi * p.groups + g) * N * ldb;
  const float* Cg = p.C + ((long long)bi * p.groups + g) * N * ldb;
  const float* Arow = p.A + (long long)d * N;
  const float bias = p.bias ? p.bias[d] : 0.0f;
  const float dskip = p.D ? p.D[d] : 0.0f;
  float* carry = small + (wave * RPW + rw) * N;
  float* a2s = small + (kWavesPerBlock * RPW + wave * RPW + rw) * N;
  float* zeros = small + 2 * kWavesPerBlock * RPW * N + kZerosPad;
  const float* cbase = j == 0 ? carry : zeros;
  const long long nch = (L + CH - 1) / CH;
  const long long nfull = L / CH;
  // this segment's full chunks [cb, ce); the last segment also runs the tail chunk
  constexpr bool segd = SEG;  // launched with p.segs > 1
  const long long cb = segd ? seg * p.seg_chunks : 0;
  const long long ce = segd ? (cb + p.seg_chunks < nfull ? cb + p.seg_chunks : nfull) : nfull;
  const bool last_seg = !segd || seg == p.segs - 1;
  // the row's 16 lanes take a state each: the state entering the segment is h0
  // through the maps of the segments before it
  for (int n = j; n < N; n += LPR) {
    float h = p.h0 ? p.h0[row * N + n] : 0.0f;
    for (int s2 = 0; SEG && s2 < seg; ++s2) {
      const float2 mp = *reinterpret_cast<const float2*>(
          p.segmap + ((row * (p.segs - 1) + s2) * N + n) * 2);
      h = fmaf(mp.x, h, mp.y);
    }
    carry[n] = h;
    a2s[n] = Arow[n] * kLog2e;
  }
  for (int i = threadIdx.x; i < N; i += blockDim.x) zeros[i] = 0.0f;

  const int ng = (N + kTileStates - 1) / kTileStates;  // tiles per chunk
  const long long cl = (TAIL && last_seg && nfull < nch) ? ce + 1 : ce;  // with the tail chunk
  const long long ntiles = (cl - cb) * ng;
  auto mem0 = [&](long long c) { return REV ? L - (c + 1) * CH : c * CH; };
  if (ntiles > 0)
    issue_tile<I, DWBC>(tiles, Bg, Cg, L, ldb, p.bpo, mem0(cb), 0, N, wave, lane,
                        TAIL && cb >= nfull);
  // In a segment (one or a few chunks per block) the first tile's sync comes after
  // the first chunk's delta/u loads, in the loop, so that their latencies overlap.
  if (!segd || cl == cb) tile_sync();

  // A lane block of a contiguous row. Aligned rows: 16-byte pieces, where in the
  // tail chunk a piece past the row's end (L % 4 == 0: a piece lies wholly in or
  // out) reads kZeroPiece; otherwise single floats, bounds-checked in the tail.
  auto load_c = [&](const float* r, long long sbl, bool full, float (&v)[I]) {
    if constexpr (ALN) {
      const long long mb = REV ? L - sbl - I : sbl;  // the block's lowest memory step
#pragma unroll
      for (int q = 0; q < I / 4; ++q) {
        const long long m = mb + 4 * q;
        const bool in = full || (REV ? m >= 0 : m < L);
        const float4 x = *reinterpret_cast<const float4*>(in ? r + m : kZeroPiece);
        const float w[4] = {x.x, x.y, x.z, x.w};
#pragma unroll
        for (int e = 0; e < 4; ++e) v[REV ? I - 1 - (4 * q + e) : 4 * q + e] = w[e];
      }
    } else {
      // one base per block and immediate offsets: traversal step sbl + i is memory
      // mb + i (forward) or mb + I-1-i (reverse)
      const float* base = r + (REV ? L - sbl - I : sbl);
#pragma unroll
      for (int i = 0; i < I; ++i)
        v[i] = full || sbl + i < L ? base[REV ? I - 1 - i : i] : 0.0f;
    }
  };

  // the lane block's outputs at traversal base sbo (SIO 0 and 1; every SIO's tail)
  auto store_out = [&](long long sbo, const float (&v)[I], bool full) {
    if (SIO && !full) {
      store_tail<I, REV>(orow, L, sbo, p.os_t, v);
    } else if (SIO) {
      const long long tlo = REV ? L - sbo - I : sbo;  // the block's lowest memory step
      store_block_strided<I, REV>(slab_rsrc(p.out + bib * p.os_b, p.o_bytes),
                                  (unsigned)((d * p.os_d + tlo * p.os_t) * 4), p.os_t, v);
    } else if constexpr (ALN) {
      const long long mb = REV ? L - sbo - I : sbo;
#pragma unroll
      for (int q = 0; q < I / 4; ++q) {
        const long long m = mb + 4 * q;
        float w[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) w[e] = v[REV ? I - 1 - (4 * q + e) : 4 * q + e];
        if (REV ? m >= 0 : m < L)  // the tail chunk: pieces inside the row only
          *reinterpret_cast<float4*>(orow + m) = make_float4(w[0], w[1], w[2], w[3]);
      }
    } else {
      // Rows that are not 16-byte multiples: the wave's four rows of the chunk pass
      // through a wave-private LDS buffer and leave with consecutive lanes storing
      // consecutive steps (whole lines), where a lane's own 16 single floats would
      // touch 16 lines 64 bytes apart (measured 186 -> 144 us at B8 D1536 L2050 with
      // 16-byte moves in place of them). The 16-byte pieces are swizzled by lane
      // block (q ^ j%4) to spread a row's writes over the banks.
      static_assert(ALN || I == 16, "the out stage holds 16 steps per lane block");
      float* wb = zbuf + wave * (RPW * CH);
#pragma unroll
      for (int q = 0; q < I / 4; ++q)
        *reinterpret_cast<float4*>(wb + rw * CH + 16 * j + 4 * (q ^ (j & 3))) =
            make_float4(v[4 * q], v[4 * q + 1], v[4 * q + 2], v[4 * q + 3]);
      const long long t0 = sbo - (long long)j * I + lane;  // this lane's first step
      // the wave's first row at step t0; rows L floats apart, steps +-64 per round
      float* ob = p.out + (blk * kWavesPerBlock + wave) * RPW * L + (REV ? L - 1 - t0 : t0);
#pragma unroll
      for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int k4 = 0; k4 < (int)CH / 64; ++k4) {
          const int ps = 64 * k4 + lane;  // step of the chunk
          const int jb = ps >> 4, i = ps & 15;
          const float val = wb[r * CH + 16 * jb + 4 * ((i >> 2) ^ (jb & 3)) + (i & 3)];
          if (full || t0 + 64 * k4 < L) ob[r * L + (REV ? -64 * k4 : 64 * k4)] = val;
        }
    }
  };

  // SIO 2, 3: chunk c's z stage is issued once chunk c-1's outputs have left the stage
  // (a sync), lands by chunk c's first tile sync (ng >= 2) and is read after chunk
  // c's last tile's states.
  const int d0 = (int)(blk * (kWavesPerBlock * RPW) % p.dim);  // the block's first channel
  auto z_stage = [&](long long c) {
    issue_z_stage<REV>(zbuf, p.z + bib * p.zs_b, p.zs_t, L, c * CH, d0, wave, lane,
                       TAIL && c >= nfull);
  };
  // u through the stage too: per chunk, u's DMA, its read, then z's DMA
  constexpr bool ustage = SIO == 3;
  if (SIO == 2 && p.z && cl > cb) z_stage(cb);

  long long k = 0;  // tile counter
  // One chunk; FULL: every step inside the row. The tail chunk is its own compiled
  // copy, so that its bounds checks hold no registers in the loop over whole chunks.
  auto run_chunk = [&](long long c, auto full_tag) {
    constexpr bool full = decltype(full_tag)::value;
    const long long sb = c * CH + (long long)j * I;
    float dt[I], du[I], y[I], zz[I];
    float sdt = 0.0f;
    {
      float dd[I], uu[I];
      load_c(drow, sb, full, dd);
      if (ustage) {
        if constexpr (SIO == 3) {
          // the block's 16 channels of u, 64-byte runs, land with delta's loads; the
          // stage is free (the previous chunk's outputs have left it) and z's DMA
          // follows once every lane has read its u
          issue_z_stage<REV>(zbuf, p.u + bib * p.us_b, p.us_t, L, c * CH, d0, wave, lane,
                             !full);
          tile_sync();
          read_z_stage(zbuf, j, wave, rw, uu);
          lds_barrier();
          if (p.z) z_stage(c);
        }
      } else if (ustr && !full) {
        load_tail<I, REV>(urow, L, sb, p.us_t, uu);
      } else if (ustr) {
        const long long tlo = REV ? L - sb - I : sb;  // the block's lowest memory step
        load_block_strided<I, REV>(slab_rsrc(p.u + bib * p.us_b, p.u_bytes),
                                   (unsigned)((d * p.us_d + tlo * p.us_t) * 4), p.us_t, uu);
      } else {
        load_c(urow, sb, full, uu);
      }
#pragma unroll
      for (int i = 0; i < I; ++i) {
        float x = dd[i] + bias;
        if (p.softplus) x = softplus_fast(x);
        if (!full) x = sb + i < L ? x : 0.0f;  // steps past the row: identity maps
        dt[i] = x;
        du[i] = x * uu[i];
        y[i] = dskip * uu[i];
        sdt += x;
      }
    }
    if (segd && c == cb) tile_sync();  // the first tile, the carries and A*log2e above
    const bool last_chunk = c + 1 == nch;
    for (int q = 0; q < ng; ++q, ++k) {
      progress_prio(k, ntiles);
      if (k + 1 < ntiles) {  // the next tile: state group q + 1 of this chunk, or 0 of the next
        const bool same = q + 1 < ng;
        const long long cn = same ? c : c + 1;
        issue_tile<I, DWBC>(tiles + ((k + 1) & 1) * G::FLOATS, Bg, Cg, L, ldb, p.bpo, mem0(cn),
                            same ? (q + 1) * kTileStates : 0, N, wave, lane,
                            TAIL && cn >= nfull);
      }
      if (SIO == 1 && !full && zrow && q + 1 == ng) {
        load_tail<I, REV>(zrow, L, sb, p.zs_t, zz);
      } else if (SIO < 2 && zrow && q + 1 == ng) {
        if (SIO == 1) {
          const long long tlo = REV ? L - sb - I : sb;  // the block's lowest memory step
          load_block_strided<I, REV>(slab_rsrc(p.z + bib * p.zs_b, p.z_bytes),
                                     (unsigned)((d * p.zs_d + tlo * p.zs_t) * 4), p.zs_t, zz);
        } else {
          load_c(zrow, sb, full, zz);
        }
      }
      tile_states<I, REV>(tiles + (k & 1) * G::FLOATS, q * kTileStates, N, j, a2s, cbase,
                          carry, (last_chunk && p.last) ? p.last + row * N : nullptr, dt, du,
                          sdt, y);
      if (SIO >= 2 && zrow && q + 1 == ng) {
        // after the states (no registers held through them), before the sync after
        // which the outputs overwrite it
        static_assert(SIO < 2 || I == 16, "the stage holds 16 steps per lane block");
        read_z_stage(zbuf, j, wave, rw, zz);
      }
      tile_sync();
    }
    if (zrow) {
#pragma unroll
      for (int i = 0; i < I; ++i) y[i] *= silu_fast(zz[i]);
    }
    if constexpr (SIO >= 2) {
      write_out_stage(zbuf, j, wave, rw, y);
      lds_barrier();
      store_out_stage<REV>(zbuf, p.out + bib * p.os_b, p.os_t, L, c * CH, d0, wave, lane,
                           !full);
      lds_barrier();  // every lane has read its outputs before the next z stage lands
      if (p.z && c + 1 < cl && !ustage) z_stage(c + 1);
    } else {
      store_out(sb, y, full);
    }
  };
  for (long long c = cb; c < ce; ++c) run_chunk(c, std::true_type{});
  if constexpr (TAIL)
    if (cl > ce) run_chunk(ce, std::false_type{});
}

// Pass 1 of a segmented scan: the affine map h -> A h + B of each state over one
// segment of 16 rows (segments 0 .. segs-2), with the same discretisation and
// fold as tile_state; the chunk maps compose in order. A of a chunk is
// 2^(a2 * sum of the row's dt over it), one exponential.
template <int I, bool REV, bool ALN = true, bool DWBC = !ALN>
__device__ __forceinline__ void fold_rows(const M1Kern& p, long long blk, int seg) {
  constexpr int LPR = 16, RPW = 4;
  using G = Tile<I>;
  constexpr long long CH = G::CH;
  extern __shared__ __attribute__((aligned(16))) float s_lds[];
  float* tiles = s_lds;                  // [2][G::FLOATS]
  float* small = s_lds + 2 * G::FLOATS;  // segment A, B, A*log2e per row and state

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int j = lane % LPR;
  const int rw = lane / LPR;
  const long long row = (blk * kWavesPerBlock + wave) * RPW + rw;
  const long long L = p.L;
  const int N = p.N;
  const int bi = (int)(row / p.dim), d = (int)(row - (long long)bi * p.dim);
  const int g = d / p.group_size;
  const float* urow = p.u + row * L;
  const float* drow = p.delta + row * L;
  // strided u (the seam kernels): the block's 16 rows share one batch, wave-uniform
  const long long bib = blk * (kWavesPerBlock * RPW) / p.dim;
  const long long ldb = p.ldb;
  const float* Bg = p.B + ((long long)bi * p.groups + g) * N * ldb;
  const float bias = p.bias ? p.bias[d] : 0.0f;
  float* sA = small + (wave * RPW + rw) * N;
  float* sB = small + (kWavesPerBlock * RPW + wave * RPW + rw) * N;
  float* a2s = small + (2 * kWavesPerBlock * RPW + wave * RPW + rw) * N;
  for (int n = j; n < N; n += LPR) {
    sA[n] = 1.0f;
    sB[n] = 0.0f;
    a2s[n] = p.A[(long long)d * N + n] * kLog2e;
  }

  const long long nfull = L / CH;
  const long long cb = seg * p.seg_chunks;
  const long long ce = cb + p.seg_chunks < nfull ? cb + p.seg_chunks : nfull;
  const int ng = (N + kTileStates - 1) / kTileStates;
  const long long ntiles = (ce - cb) * ng;
  auto mem0 = [&](long long c) { return REV ? L - (c + 1) * CH : c * CH; };
  // the fold reads B only: the tiles' C rows are not fetched
  if (ntiles > 0)
    issue_tile<I, DWBC>(tiles, Bg, nullptr, L, ldb, p.bpo, mem0(cb), 0, N, wave, lane);
  long long k = 0;
  for (long long c = cb; c < ce; ++c) {
    const long long sb = c * CH + (long long)j * I;
    float dt[I], du[I];
    float sdt = 0.0f;
    {
      float dd[I], uu[I];
      // the segments folded here hold whole chunks: no bounds to check
      load_block<I, REV, ALN>(drow, sb + I, sb, 0.0f, dd, L);
      if (ALN && p.u_strided) {
        const long long tlo = REV ? L - sb - I : sb;  // the block's lowest memory step
        load_block_strided<I, REV>(slab_rsrc(p.u + bib * p.us_b, p.u_bytes),
                                   (unsigned)((d * p.us_d + tlo * p.us_t) * 4), p.us_t, uu);
      } else {
        load_block<I, REV, ALN>(urow, sb + I, sb, 0.0f, uu, L);
      }
#pragma unroll
      for (int i = 0; i < I; ++i) {
        float x = dd[i] + bias;
        if (p.softplus) x = softplus_fast(x);
        dt[i] = x;
        du[i] = x * uu[i];
        sdt += x;
      }
    }
    if (c == cb) tile_sync();  // the first tile, and the initial maps above
    float srow = sdt;  // the row's dt over the chunk
#pragma unroll
    for (int m = 1; m < LPR; m <<= 1) srow += __shfl_xor(srow, m, LPR);
    for (int q = 0; q < ng; ++q, ++k) {
      progress_prio(k, ntiles);
      if (k + 1 < ntiles) {  // the next tile: state group q + 1 of this chunk, or 0 of the next
        const bool same = q + 1 < ng;
        issue_tile<I, DWBC>(tiles + ((k + 1) & 1) * G::FLOATS, Bg, nullptr, L, ldb, p.bpo,
                            mem0(same ? c : c + 1), same ? (q + 1) * kTileStates : 0, N, wave,
                            lane);
      }
      const float* tile = tiles + (k & 1) * G::FLOATS;
#pragma unroll
      for (int s2 = 0; s2 < kTileStates; ++s2) {
        const int n = q * kTileStates + s2;
        if (n < N) {
          float bb[I];
          lds_block<I, REV>(tile + s2 * CH, j, bb);
          const float a2 = a2s[n];
          float bt = 0.0f;
#pragma unroll
          for (int i = 0; i < I; ++i) bt = fmaf(ex2(dt[i] * a2), bt, du[i] * bb[i]);
          float at = ex2(a2 * sdt);
          Row<16>::scan(at, bt);  // lane 15: the chunk's B from a zero state
          if (j == LPR - 1) {
            const float ac = ex2(a2 * srow);
            sB[n] = fmaf(ac, sB[n], bt);
            sA[n] = ac * sA[n];
          }
        }
      }
      tile_sync();
    }
  }
  if (j == LPR - 1)
    for (int n = 0; n < N; ++n) {
      float* mp = p.segmap + ((row * (p.segs - 1) + seg) * N + n) * 2;
      mp[0] = sA[n];
      mp[1] = sB[n];
    }
}

template <int I, bool REV, bool ALN, bool DWBC>
__global__ void __launch_bounds__(64 * kWavesPerBlock, 3)
m1_seg_fold_kernel(M1Kern p) {
  const long long nblk = p.rows / (kWavesPerBlock * 4);
  fold_rows<I, REV, ALN, DWBC>(p, blockIdx.x % nblk, (int)(blockIdx.x / nblk));
}

// Rows of B or C copied to a row pitch of ldb floats (ldb >= L), each row's data
// starting `off` floats in and zeros around it, so that the tiled kernel moves them
// by 16-byte DMA.
__global__ void __launch_bounds__(256) pad_rows_kernel(const float* __restrict__ src,
                                                       float* __restrict__ dst, long long rows,
                                                       long long L, long long ldb,
                                                       long long off) {
  const long long e = (long long)blockIdx.x * blockDim.x + threadIdx.x;
  if (e >= rows * ldb) return;
  const long long r = e / ldb, t = e - r * ldb - off;
  dst[e] = t >= 0 && t < L ? src[r * L + t] : 0.0f;
}

// Block id -> row block for time-major z/out: a 128-byte line of those holds 32
// channels, two row blocks' worth, so adjacent row blocks go to one XCD (block id
// mod 8), dispatched back to back, and each line is fetched and written back whole
// by one L2. Ids past the last multiple of 16 map to themselves.
__device__ __forceinline__ long long paired_block(long long bid, long long nblk) {
  if (bid >= (nblk & ~15LL)) return bid;
  const long long x = bid & 7, k = bid >> 3;
  return 2 * (8 * (k >> 1) + x) + (k & 1);
}

// Block id -> (row block, segment): with SEG the segments are blockIdx / (row blocks).
template <int I, bool REV, int SIO, bool SEG, bool ALN, bool TAIL, bool DWBC>
__global__ void __launch_bounds__(64 * kWavesPerBlock, 3)
m1_tile_kernel(M1Kern p) {
  const long long nblk = p.rows / (kWavesPerBlock * 4);
  const long long bid = SEG ? blockIdx.x % nblk : (long long)blockIdx.x;
  const int seg = SEG ? (int)(blockIdx.x / nblk) : 0;
  // Whole rows: each XCD (block id mod 8) takes a contiguous eighth of the row
  // blocks, dispatched in order, so the rows of one batch, which read the same B and
  // C tiles, meet in one L2, and adjacent row blocks (which share the 128-byte lines
  // of time-major z and out) run back to back on one XCD. Headline 127.2 -> 124.8 us,
  // the seam's time-major layer 146.0 -> 142.9 us, bit-identical. With a multiple of
  // 8 but not of 16 row blocks the strided kernels keep the explicit pairing.
  long long blk = bid;
  if (!SEG && nblk % 16 == 0) blk = (bid & 7) * (nblk / 8) + (bid >> 3);
  else if (SIO) blk = paired_block(bid, nblk);
  else if (!SEG && nblk % 8 == 0) blk = (bid & 7) * (nblk / 8) + (bid >> 3);
  tile_rows<I, REV, SIO, SEG, ALN, TAIL, DWBC>(p, blk, seg);
}

// Several traversals of rows of the same shape in one launch (the directions of
// a 2D cross-scan): every job has p.rows / 16 blocks. Each XCD (block id mod 8)
// takes a contiguous range of row blocks, with the jobs of a row block next to each
// other, so the row blocks of one batch, which read the same B and C tiles, share
// its L2 (at D 192 a batch is 12 row blocks; config-5 SS2D 331 -> 327 us).
template <int I, bool TAIL, bool ALN>
__global__ void __launch_bounds__(64 * kWavesPerBlock, 3)
m1_tile_jobs_kernel(M1Kern p, M1Jobs jobs) {
  const int xcd = blockIdx.x & 7;
  const int k = blockIdx.x >> 3;
  const int ji = k % jobs.njobs;
  const long long per = (jobs.blocks_per_job + 7) / 8;  // row blocks per XCD
  const long long blk = xcd * per + k / jobs.njobs;
  if (blk >= jobs.blocks_per_job) return;  // whole block: no barrier is reached
  const M1Job& jb = jobs.job[ji];
  p.u = jb.u;
  p.delta = jb.delta;
  p.z = jb.z;
  p.B = jb.B;
  p.C = jb.C;
  p.out = jb.out;
  p.last = jb.last;
  if (jb.rev) tile_rows<I, true, 0, false, ALN, TAIL>(p, blk);
  else tile_rows<I, false, 0, false, ALN, TAIL>(p, blk);
}

template <int I, bool REV, int SIO, bool ALN, bool DWBC>
hipError_t launch_tile(const M1Kern& k, hipStream_t st) {
  constexpr int RPB = kWavesPerBlock * 4;
  const long long blocks = (long long)k.rows / RPB;
  const int segs = k.segs > 1 ? k.segs : 1;
  if (segs > 1) {  // pass 1: the maps of segments 0 .. segs-2
    const size_t lds1 = sizeof(float) * (2 * (size_t)Tile<I>::FLOATS + 3 * (size_t)RPB * k.N);
    hipLaunchKernelGGL((m1_seg_fold_kernel<I, REV, ALN, DWBC>),
                       dim3((unsigned)(blocks * (segs - 1))),
                       dim3(64 * kWavesPerBlock), lds1, st, k);
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const size_t lds =
      sizeof(float) * (2 * (size_t)Tile<I>::FLOATS + (SIO >= 2 || !ALN ? kZStageFloats : 0) +
                       (2 * (size_t)RPB + 1) * k.N + kZerosPad);
  const dim3 grid((unsigned)(segs > 1 ? blocks * segs : blocks)), wg(64 * kWavesPerBlock);
  const bool tail = k.L % Tile<I>::CH != 0;
  if (segs > 1 && tail)
    hipLaunchKernelGGL((m1_tile_kernel<I, REV, SIO, true, ALN, true, DWBC>), grid, wg, lds, st,
                       k);
  else if (segs > 1)
    hipLaunchKernelGGL((m1_tile_kernel<I, REV, SIO, true, ALN, false, DWBC>), grid, wg, lds, st,
                       k);
  else if (tail)
    hipLaunchKernelGGL((m1_tile_kernel<I, REV, SIO, false, ALN, true, DWBC>), grid, wg, lds, st,
                       k);
  else
    hipLaunchKernelGGL((m1_tile_kernel<I, REV, SIO, false, ALN, false, DWBC>), grid, wg, lds,
                       st, k);
  return hipGetLastError();
}

template <int LPR, int I, bool REV, bool VEC>
hipError_t launch(const M1Kern& k, hipStream_t st) {
  constexpr int RPB = kWavesPerBlock * (64 / LPR);
  const long long blocks = ((long long)k.rows + RPB - 1) / RPB;
  const size_t lds = 2 * sizeof(float) * (size_t)kWavesPerBlock * (64 / LPR) * k.N;
  hipLaunchKernelGGL((m1_chunk_kernel<LPR, I, REV, VEC>), dim3((unsigned)blocks),
                     dim3(64 * kWavesPerBlock), lds, st, k);
  return hipGetLastError();
}

template <int LPR, int I>
hipError_t launch_dir(const M1Kern& k, bool rev, bool vec, hipStream_t st) {
  if (rev) return vec ? launch<LPR, I, true, true>(k, st) : launch<LPR, I, true, false>(k, st);
  return vec ? launch<LPR, I, false, true>(k, st) : launch<LPR, I, false, false>(k, st);
}

bool aligned16(const void* q) { return q == nullptr || ((uintptr_t)q & 15u) == 0; }

}  // namespace

// Rows of any length and alignment: unaligned ones (L % 4 != 0 or a base off 16 bytes)
// take the single-float instantiation.
bool m1_jobs_supported(const M1Problem& pr) {
  return pr.dim % 16 == 0 && pr.groups == 1 && pr.h0 == nullptr;
}

hipError_t m1_scan_jobs(const M1Problem& pr, const M1JobSpec* spec, int n, hipStream_t st) {
  if (n < 1 || n > kMaxJobs || !m1_jobs_supported(pr)) return hipErrorInvalidValue;
  M1Kern k{};
  k.A = pr.A; k.D = pr.D; k.bias = pr.bias; k.h0 = nullptr;
  k.L = (long long)pr.len; k.rows = (int)(pr.batch * pr.dim); k.dim = (int)pr.dim;
  k.ldb = k.L; k.bpo = 0;
  k.N = (int)pr.state; k.groups = 1; k.group_size = (int)pr.dim;
  k.softplus = pr.softplus;
  M1Jobs jobs{};
  jobs.njobs = n;
  jobs.blocks_per_job = k.rows / 16;
  bool aln = pr.len % 4 == 0;
  for (int i = 0; i < n; ++i) {
    const M1JobSpec& j = spec[i];
    aln = aln && aligned16(j.u) && aligned16(j.delta) && aligned16(j.z) && aligned16(j.B) &&
          aligned16(j.C) && aligned16(j.out);
    jobs.job[i] = M1Job{j.u, j.delta, j.z, j.B, j.C, j.out, j.last, j.rev};
  }
  const long long blocks = 8LL * n * ((jobs.blocks_per_job + 7) / 8);
  const size_t lds = sizeof(float) * (2 * (size_t)Tile<M1_TILE_I>::FLOATS +
                                      (aln ? 0 : kZStageFloats) + (2 * (size_t)16 + 1) * k.N +
                                      kZerosPad);
  const bool tail = k.L % Tile<M1_TILE_I>::CH != 0;
  const dim3 grid((unsigned)blocks), wg(64 * kWavesPerBlock);
  if (aln && tail)
    hipLaunchKernelGGL((m1_tile_jobs_kernel<M1_TILE_I, true, true>), grid, wg, lds, st, k, jobs);
  else if (aln)
    hipLaunchKernelGGL((m1_tile_jobs_kernel<M1_TILE_I, false, true>), grid, wg, lds, st, k, jobs);
  else if (tail)
    hipLaunchKernelGGL((m1_tile_jobs_kernel<M1_TILE_I, true, false>), grid, wg, lds, st, k, jobs);
  else
    hipLaunchKernelGGL((m1_tile_jobs_kernel<M1_TILE_I, false, false>), grid, wg, lds, st, k,
                       jobs);
  return hipGetLastError();
}

namespace {
// Strides are meaningful only with has_strides (the strided entry point writes the
// contiguous ones for a null array); without it every tensor is contiguous.
bool contiguous_strides(const long long (&s)[3], const M1Problem& pr) {
  const long long L = (long long)pr.len, D = (long long)pr.dim;
  return !pr.has_strides || (s[0] == D * L && s[1] == L && s[2] == 1);
}
// bytes of one batch's slab of a strided (batch, dim, len) tensor
long long slab_bytes(const long long (&s)[3], const M1Problem& pr) {
  return 4 * ((long long)(pr.dim - 1) * s[1] + (long long)(pr.len - 1) * s[2] + 1);
}
}  // namespace

// The allocation-free entry point's scratch (arm_scan_selective_scan_noalloc_f32):
// the segment maps of the few-rows plan live here instead of in stream-ordered
// allocations. Every device holds its own copy until the process ends; host code
// reaches it only through the address m1_noalloc_scratch looks up per device.
constexpr size_t kNoAllocScratchBytes = size_t(4) << 20;
static __device__ __align__(256) float scratch[kNoAllocScratchBytes / sizeof(float)];

hipError_t m1_noalloc_scratch(float** out, size_t* bytes) {
  constexpr int kMaxDevices = 64;
  static std::atomic<float*> addr[kMaxDevices];
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  float* p = addr[dev].load(std::memory_order_acquire);
  if (p == nullptr) {
    // with this device current: its copy of the array (racing threads find the same)
    e = hipGetSymbolAddress((void**)&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return e;
    addr[dev].store(p, std::memory_order_release);
  }
  *out = p;
  *bytes = kNoAllocScratchBytes;
  return hipSuccess;
}

namespace {
// Rows cut into segments when there are too few to fill the chip: a 16-row block per
// CU slot, 768 slots (three per CU) resident at once. Sets k.segs / k.seg_chunks and
// allocates the segment maps on the stream, or, with caller scratch, takes them from
// it, cutting the plan to fewer segments (down to whole rows, which need no maps)
// until they fit.
hipError_t plan_segments(M1Kern& k, float* scratch_p, size_t scratch_bytes, hipStream_t st) {
  static_assert(16 * M1_TILE_I == kM1ChunkSteps, "chunk size shared with the ABI's routing");
  const long long blocks = k.rows / 16;
  const long long nfull = k.L / (16 * M1_TILE_I);
  k.segs = 1;
  k.seg_chunks = nfull;
  k.segmap = nullptr;
  if (blocks >= kM1WholeRowBlocks || nfull < 2) return hipSuccess;
  long long segs = (768 + blocks - 1) / blocks;
  if (segs > nfull) segs = nfull;
  auto map_bytes = [&](long long s) {
    return (size_t)k.rows * (size_t)(s - 1) * (size_t)k.N * 2 * sizeof(float);
  };
  if (scratch_p)
    while (segs >= 2 && map_bytes(segs) > scratch_bytes) --segs;
  if (segs < 2) return hipSuccess;
  k.seg_chunks = (nfull + segs - 1) / segs;
  k.segs = (int)((nfull + k.seg_chunks - 1) / k.seg_chunks);
  if (k.segs < 2) {
    k.segs = 1;
    k.seg_chunks = nfull;
    return hipSuccess;
  }
  if (scratch_p) {
    k.segmap = scratch_p;  // every map is written by the fold before the replay reads it
    return hipSuccess;
  }
  return stream_alloc((void**)&k.segmap, map_bytes(k.segs), st);
}

template <int SIO, bool ALN = true, bool DWBC = false>
hipError_t run_tile(M1Kern& k, bool rev, float* scratch_p, size_t scratch_bytes,
                    hipStream_t st) {
  hipError_t e = plan_segments(k, scratch_p, scratch_bytes, st);
  if (e != hipSuccess) return e;
  e = rev ? launch_tile<M1_TILE_I, true, SIO, ALN, DWBC>(k, st)
          : launch_tile<M1_TILE_I, false, SIO, ALN, DWBC>(k, st);
  if (k.segmap && !scratch_p) {
    const hipError_t fe = hipFreeAsync(k.segmap, st);
    if (e == hipSuccess) e = fe;
  }
  return e;
}
}  // namespace

bool m1_strided_io(const M1Problem& pr) {
  return (pr.z && !contiguous_strides(pr.z_stride, pr)) ||
         !contiguous_strides(pr.out_stride, pr) || !contiguous_strides(pr.u_stride, pr);
}

// Whether a strided (batch, dim, len) layout gives every element its own address:
// with the dimensions of more than one element sorted by stride, each stride must
// step past the whole extent of the smaller ones. (This also rejects some exotic
// interleavings that do not overlap; no tensor view produces those.)
bool distinct_elements(const long long (&s)[3], const M1Problem& pr) {
  const long long n[3] = {(long long)pr.batch, (long long)pr.dim, (long long)pr.len};
  int ord[3], k = 0;
  for (int i = 0; i < 3; ++i)
    if (n[i] > 1) ord[k++] = i;
  for (int a = 1; a < k; ++a)  // insertion sort by stride
    for (int b = a; b > 0 && s[ord[b]] < s[ord[b - 1]]; --b) std::swap(ord[b], ord[b - 1]);
  long long extent = 0;  // largest offset reached by the smaller dimensions
  for (int a = 0; a < k; ++a) {
    const int i = ord[a];
    if (s[i] <= extent) return false;
    extent += s[i] * (n[i] - 1);
  }
  return true;
}

bool m1_strided_supported(const M1Problem& pr, const char** why) {
  auto no = [&](const char* w) {
    if (why) *why = w;
    return false;
  };
  const bool u_cont = contiguous_strides(pr.u_stride, pr);
  if (pr.len % 4 != 0 || (u_cont && !aligned16(pr.u)) || !aligned16(pr.delta) ||
      !aligned16(pr.B) || !aligned16(pr.C))
    return no("strided z/out need len % 4 == 0 and 16-byte aligned u, delta, B, C");
  if (pr.dim % 16 != 0 || (pr.dim / pr.groups) % 16 != 0)
    return no("strided z/out need dim and dim/groups multiples of 16");
  for (int t = 0; t < 3; ++t) {
    const long long(&s)[3] = t == 2 ? pr.u_stride : t ? pr.out_stride : pr.z_stride;
    if (t == 0 && !pr.z) continue;
    if (contiguous_strides(s, pr)) continue;
    if (s[0] < 0 || s[1] < 0 || s[2] < 0) return no("negative z/out/u strides");
    if (t == 1 && !distinct_elements(s, pr))
      return no("out strides make elements overlap (a zero or too small stride)");
    if (slab_bytes(s, pr) >= (1LL << 32) || 4LL * (M1_TILE_I - 1) * s[2] >= (1LL << 31))
      return no("a batch of strided z/out/u must span less than 4 GiB");
  }
  return true;
}

hipError_t m1_scan_chunked(const M1Problem& pr, hipStream_t st) {
  M1Kern k{};
  k.u = pr.u; k.delta = pr.delta; k.A = pr.A; k.B = pr.B; k.C = pr.C; k.D = pr.D; k.z = pr.z;
  k.bias = pr.bias; k.h0 = pr.h0; k.out = pr.out; k.last = pr.last;
  k.L = (long long)pr.len; k.rows = (int)(pr.batch * pr.dim); k.dim = (int)pr.dim;
  k.ldb = k.L; k.bpo = 0;
  k.N = (int)pr.state; k.groups = (int)pr.groups; k.group_size = (int)(pr.dim / pr.groups);
  k.softplus = pr.softplus;
  const bool vec = pr.len % 4 == 0 && aligned16(pr.u) && aligned16(pr.delta) &&
                   aligned16(pr.B) && aligned16(pr.C) && aligned16(pr.z) && aligned16(pr.out);
  const bool rev = pr.reverse != 0;
  if (m1_strided_io(pr)) {
    if (!m1_strided_supported(pr, nullptr)) return hipErrorInvalidValue;
    const long long L = (long long)pr.len, D = (long long)pr.dim;
    const long long zc[3] = {D * L, L, 1};
    const bool zcont = contiguous_strides(pr.z_stride, pr), ocont = contiguous_strides(pr.out_stride, pr);
    const long long(&zs)[3] = zcont ? zc : pr.z_stride;
    const long long(&os)[3] = ocont ? zc : pr.out_stride;
    k.zs_b = zs[0]; k.zs_d = zs[1]; k.zs_t = zs[2];
    k.os_b = os[0]; k.os_d = os[1]; k.os_t = os[2];
    k.z_bytes = pr.z ? (unsigned)slab_bytes(zs, pr) : 0u;
    // the LDS stage: 16-byte channel runs of out (and z), and for z a chunk of at
    // least two tiles between issuing the stage and reading it
    k.z_dma = os[1] == 1 && os[2] % 4 == 0 && os[0] % 4 == 0 && aligned16(pr.out) &&
              (!pr.z || (zs[1] == 1 && zs[2] % 4 == 0 && zs[0] % 4 == 0 && aligned16(pr.z) &&
                         pr.state > kTileStates)) &&
              M1_TILE_I == 16;
    k.o_bytes = (unsigned)slab_bytes(os, pr);
    if (!contiguous_strides(pr.u_stride, pr)) {
      k.u_strided = 1;
      k.us_b = pr.u_stride[0]; k.us_d = pr.u_stride[1]; k.us_t = pr.u_stride[2];
      k.u_bytes = (unsigned)slab_bytes(pr.u_stride, pr);
      k.u_dma = k.z_dma && k.us_d == 1 && k.us_t % 4 == 0 && k.us_b % 4 == 0 &&
                aligned16(pr.u);
    }
    if (k.z_dma)
      return k.u_dma ? run_tile<3>(k, rev, pr.scratch, pr.scratch_bytes, st)
                     : run_tile<2>(k, rev, pr.scratch, pr.scratch_bytes, st);
    return run_tile<1>(k, rev, pr.scratch, pr.scratch_bytes, st);
  }
  // the tiled path needs every 16-row block inside one batch/group
  const bool tiled = pr.dim % 16 == 0 && (pr.dim / pr.groups) % 16 == 0;
  if (!tiled) return launch_dir<16, 16>(k, rev, vec, st);
  if (vec) return run_tile<0, true>(k, rev, pr.scratch, pr.scratch_bytes, st);
  // Rows that are not 16-byte multiples: u, delta, z and out move as single floats.
  // B and C (shared by every channel, a few MB) are copied to a row pitch rounded up
  // to 4 so that the tiles still fill by 16-byte DMA (B8 D1536 L2050: 209 -> 187 us
  // with 16-byte DMA). The allocation-free entry, which owns no memory for the copy,
  // moves them as single floats instead.
  if (k.L % 4 == 0 && aligned16(pr.B) && aligned16(pr.C))
    return run_tile<0, false, false>(k, rev, pr.scratch, pr.scratch_bytes, st);
  if (pr.scratch) return run_tile<0, false, true>(k, rev, pr.scratch, pr.scratch_bytes, st);
  const long long ldb = (k.L + 3) & ~3LL;
  const long long off = rev ? ldb - k.L : 0;  // reverse chunks end at L: pad in front
  const long long bcrows = (long long)pr.batch * pr.groups * pr.state;
  const long long n = bcrows * ldb;
  float* pad = nullptr;
  hipError_t e = stream_alloc((void**)&pad, 2 * (size_t)n * sizeof(float), st);
  if (e != hipSuccess) return e;
  const unsigned pblocks = (unsigned)((n + 255) / 256);
  hipLaunchKernelGGL(pad_rows_kernel, dim3(pblocks), dim3(256), 0, st, pr.B, pad, bcrows, k.L,
                     ldb, off);
  hipLaunchKernelGGL(pad_rows_kernel, dim3(pblocks), dim3(256), 0, st, pr.C, pad + n, bcrows,
                     k.L, ldb, off);
  e = hipGetLastError();
  if (e == hipSuccess) {
    k.B = pad + off;  // each row's first data float
    k.C = pad + n + off;
    k.ldb = ldb;
    k.bpo = off;
    e = run_tile<0, false, false>(k, rev, nullptr, 0, st);
  }
  const hipError_t fe = hipFreeAsync(pad, st);
  return e != hipSuccess ? e : fe;
}

}  // namespace armscan
