// Host-side launchers behind the C ABI (internal to libarm_scan_hip.so).
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>

namespace armscan {

// One Mamba-1 problem: the reference's layouts (lib.rs:9-16) on device memory.
struct M1Problem {
  size_t batch, dim, len, state, groups;
  const float *u, *delta, *A, *B, *C;
  const float *B2, *C2;  // backward-direction B/C for the bidirectional pass (null = B/C)
  const float *D, *z, *bias, *h0;
  float *out, *last;
  float *out2, *last2;  // bidirectional outputs
  int softplus, reverse;
  int merge;  // bidirectional: write out = fwd + bwd instead of two outputs
  // Element strides (batch, dim, step) of z, out and u, read only when has_strides is
  // set (the strided entry point, which writes the contiguous (dim*len, len, 1) for a
  // null stride array). Every value is taken as given: a stride of 0 is a broadcast.
  int has_strides;
  long long z_stride[3], out_stride[3], u_stride[3];
  // Caller-provided scratch for the segment maps of the few-rows plan (the
  // allocation-free entry point passes its static device array): when set, nothing
  // is allocated, and the plan is cut to what scratch_bytes holds.
  float* scratch;
  size_t scratch_bytes;
};

hipError_t m1_scan(const M1Problem& p, hipStream_t st);
// The per-device address and size of the allocation-free entry point's static scratch
// (m1_chunk.hip), looked up once per device with that device current.
hipError_t m1_noalloc_scratch(float** p, size_t* bytes);

// One decode step of the Mamba-1 scan, the state (batch, dim, N) updated in place
// (m1_step.hip). Element strides: x, dt, z (batch, dim); B, C (batch, state).
struct M1Step {
  float* state;
  const float *x, *dt, *A, *B, *C, *D, *z, *bias;
  float* out;  // (batch, dim)
  long long xs[2], dts[2], zs[2], Bs[2], Cs[2];
  int batch, dim, N, softplus;
};
hipError_t m1_step(const M1Step& p, hipStream_t st);
// True when z or out has strides other than the contiguous (batch, dim, len) ones.
bool m1_strided_io(const M1Problem& p);
// Whether the one-direction scan serves the strides of z/out; else *why says what fails.
bool m1_strided_supported(const M1Problem& p, const char** why);
// One direction through the chunked DPP-scan kernel (m1_chunk.hip).
hipError_t m1_scan_chunked(const M1Problem& p, hipStream_t st);
// True when the fused bidirectional kernel can hold a whole row in one pass.
bool m1_bidir_fusable(const M1Problem& p);
// Up to four traversals of rows of one shape in one launch (m1_chunk.hip), each
// with its own u/delta/z rows, B/C, output, final state and direction; rows of
// 4k floats, 16-byte aligned, dim % 16 == 0, one B/C group, no h0.
struct M1JobSpec {
  const float *u, *delta, *z, *B, *C;
  float *out, *last;
  int rev;
};
// Steps per chunk of the tiled Mamba-1 kernel (16 lanes of 16 steps a row), and the
// row blocks (16 rows each) at which a launch stops cutting rows into segments.
constexpr long long kM1ChunkSteps = 256;
constexpr long long kM1WholeRowBlocks = 512;
// blocks from which a multi-traversal launch of whole rows is preferred (one per CU)
constexpr long long kM1JobsMinBlocks = 256;
bool m1_jobs_supported(const M1Problem& p);
hipError_t m1_scan_jobs(const M1Problem& p, const M1JobSpec* spec, int n, hipStream_t st);
// Batched (planes, H, W) -> (planes, W, H) transposes of up to 8 tensors.
struct TransposeSpec {
  const float* in;
  float* out;
  long long planes;
};
hipError_t transpose_batch(const TransposeSpec* spec, int n, int H, int W, hipStream_t st);
// out = scale * (out + p1 + T(q2) + T(q3)) over (planes, H, W), with q2/q3 given as
// (planes, W, H): the merge of a 2D cross-scan whose column planes are transposed.
hipError_t merge4_transposed(float* out, const float* p1, const float* q2, const float* q3,
                             long long planes, int H, int W, float scale, hipStream_t st);
hipError_t m1_bidir(const M1Problem& p, hipStream_t st);
// (planes, H, W) -> (planes, W, H); accumulate adds into `out`.
hipError_t transpose_hw(const float* in, float* out, long long planes, int H, int W,
                        bool accumulate, hipStream_t st);
hipError_t scale_inplace(float* x, long long n, float scale, hipStream_t st);
hipError_t add_inplace(float* x, const float* y, long long n, hipStream_t st);


// One Mamba-3 problem: mamba3/mod.rs:47-57 plus the groups axis on q/k.
struct M3Problem {
  size_t batch, heads, dv, dqk, len, rank, groups;
  const float *q, *k, *v, *adt, *dt, *trap, *q_bias, *k_bias, *cos, *sin, *D, *z;
  const float *psi, *zeta, *phi;  // all null = SISO
  float *out, *last_state, *last_bx;
  int reverse;
  int out_time_major;  // out (b, l, h, dv) instead of head-major (b, h, l, dv)
  // raw angles (b, l, h, n_angles) in place of cos/sin: the pre-pass fused
  const float* angles;
  size_t n_angles;
  // SISO only: leave the same-step term (gamma q.k + D) out of every output and add
  // the result to what out already holds. Run as the second traversal after the
  // other direction has written out, that gives the non-causal sum
  // forward + backward - diagonal (python/arm_scan/mamba3_noncausal.py:89-98).
  int accumulate;
  // Element strides of v and z (batch, step) and of the raw angles (batch, step,
  // head). Within a step the heads of v and z lie dv apart; the angles' head stride
  // may be 0 (one set shared by every head). m3_contiguous_strides writes the
  // contiguous layouts; the strided entry point then puts the caller's strides in,
  // each taken as given (0 is a broadcast).
  long long v_strides[2], z_strides[2], ang_strides[3];
};

inline void m3_contiguous_strides(M3Problem& p) {
  const long long L = (long long)p.len, H = (long long)p.heads;
  p.v_strides[0] = p.z_strides[0] = L * H * (long long)p.dv;
  p.v_strides[1] = p.z_strides[1] = H * (long long)p.dv;
  p.ang_strides[0] = L * H * (long long)p.n_angles;
  p.ang_strides[1] = H * (long long)p.n_angles;
  p.ang_strides[2] = (long long)p.n_angles;
}

// Largest dv * dqk the Mamba-3 kernel holds on chip.
size_t m3_max_state();
hipError_t m3_scan(const M3Problem& p, hipStream_t st);
// The RoPE angle pre-pass: angles (batch, len, heads, r), dt (batch, heads, len) ->
// cos, sin (batch, len, heads, half), theta = cumsum_len(tanh(angle) pi dt), pairs past
// r the identity (m3_angles.hip). ang_strides (batch, step, head) in elements, or null
// for the contiguous layout.
hipError_t m3_angles_to_cos_sin(const float* angles, const float* dt, size_t batch,
                                size_t len, size_t heads, size_t r, size_t half, float* cos,
                                float* sin, hipStream_t st,
                                const long long* ang_strides = nullptr);
// The Mamba-1 mixer's depthwise causal convolution (m1_conv.hip): x any strided
// (batch, dim, len) view, weight (dim, width), bias (dim) or null, silu or identity;
// out (batch, dim, len) contiguous.
struct CausalConv {
  const float* x;
  long long xs[3];  // element strides of x: batch, dim, step
  const float *w, *bias;
  float* out;
  int batch, dim, width, silu;
  long long len;
  int vec;     // set by causal_conv1d: 16-byte channel pieces
  int out_tm;  // out as (batch, len, dim) storage instead of (batch, dim, len)
};
hipError_t causal_conv1d(const CausalConv& p, hipStream_t st);
// One decode step of it: state (batch, dim, width) contiguous, the window of the last
// width inputs, shifted left in place with x (batch, dim; strides xs) appended; out
// (batch, dim) = act(bias + sum_k w[d, k] state[b, d, k]) after the shift.
struct CausalConvStep {
  const float* x;
  long long xs[2];  // element strides of x: batch, dim
  float* state;
  const float *w, *bias;
  float* out;
  int batch, dim, width, silu;
};
hipError_t causal_conv1d_step(const CausalConvStep& p, hipStream_t st);

// The Mamba-3 mixer's front-end (m3_block.hip, apps/mamba3_lm/block.py:146-178): from
// the in_proj output, the head-major gates and the RMS-normalised q (C) and k (B).
struct M3Frontend {
  const float* proj;     // (batch, len, row_stride): [z | x | B | C | dd_dt | dd_A | trap | ...]
  long long row_stride;  // floats between tokens
  int batch, len, heads, headdim, d_state, rank, groups;
  const float *dt_bias, *b_norm, *c_norm;  // (heads), (d_state), (d_state)
  float a_floor, eps;
  float *q, *k;               // (batch, len, rank, groups, d_state)
  float *adt, *dt, *trap;     // (batch, heads, len)
};
hipError_t m3_frontend(const M3Frontend& p, hipStream_t st);

// Whether m3_scan serves raw angles for this problem (the chunked kernel, forward,
// n_angles a multiple of 4 up to dqk/2, 16-byte aligned inputs); else *why says why.
bool m3_angles_supported(const M3Problem& p, const char** why);
// One workgroup per (batch, head), step by step (any shape).
hipError_t m3_scan_sequential(const M3Problem& p, hipStream_t st);
// The chunked MFMA path (m3_chunk.hip): dv, dqk multiples of 16, rank 1/2/4.
bool m3_chunk_supported(const M3Problem& p);
hipError_t m3_scan_chunked(const M3Problem& p, hipStream_t st);

// Stream-ordered scratch from the device's default pool, whose release threshold
// is raised once per device so that freed blocks stay cached between calls.
hipError_t stream_alloc(void** p, size_t bytes, hipStream_t st);

}  // namespace armscan
