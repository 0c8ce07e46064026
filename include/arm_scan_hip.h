/*
 * arm_scan_hip.h — C ABI of libarm_scan_hip.so, the MI355X (gfx950) selective-scan
 * engine that replaces the scan path of AdityaP9116/ARMHackathon ("Arm Scan").
 *
 * The entry points keep the reference's names, argument order and return codes
 * (kernel/arm-scan-ffi/src/lib.rs). What changes, as the reference's own versioning
 * rule demands (arm-scan-ffi/src/lib.rs:25-37: "bump on any signature or semantic
 * change"), is ABI 7 -> 9:
 *
 *   - every tensor pointer is a DEVICE pointer (HBM of the current HIP device);
 *   - every entry point takes a trailing `void* stream` (a hipStream_t; NULL is the
 *     null stream). The call enqueues the kernels on that stream and returns without
 *     synchronising: outputs are ready when the stream reaches that point;
 *   - ArmMamba3Dims gains `groups` (q/k carry a groups axis, head h reads group
 *     h / (heads / groups); groups == 1 is the reference layout);
 *   - Mamba-3 MIMO may write `last_state` (the reference rejects any MIMO carry);
 *   - new entry points, each described at its declaration:
 *       arm_scan_ss2d_f32, the fused four-direction 2D scan;
 *       arm_scan_selective_scan_strided_f32 and arm_scan_mamba3_scan_time_major_f32,
 *         variants for callers' layouts;
 *       arm_scan_mamba3_scan_angles_f32 and arm_scan_mamba3_angles_f32, the Mamba-3
 *         angle pre-pass fused into the scan and alone;
 *       arm_scan_selective_state_update_f32, the Mamba-1 decode step;
 *       arm_scan_causal_conv1d_f32 and arm_scan_causal_conv1d_update_f32, the Mamba-1
 *         mixer's causal convolution and its decode step;
 *       arm_scan_mamba3_noncausal_f32, the non-causal Mamba-3 sum;
 *       arm_scan_mamba3_block_frontend_f32 and arm_scan_mamba3_scan_strided_f32, the
 *         Mamba-3 mixer's front-end and the scan reading its projection in place;
 *   - code 6 reports a HIP launch / device error; arm_scan_last_error() explains
 *     the most recent nonzero code on the calling thread.
 *
 * Layouts are the reference's (row-major, contiguous, fp32):
 *   Mamba-1   u, delta, z, out (batch, dim, len); a (dim, state);
 *             b, c (batch, groups, state, len); d_skip, delta_bias (dim);
 *             last_state, h0 (batch, dim, state)
 *   Mamba-3   q, k (batch, len, rank, groups, dqk); v, z (batch, len, heads, dv);
 *             adt, dt, trap (batch, heads, len); cos, sin (batch, len, heads, dqk/2);
 *             q_bias, k_bias (heads, rank, dqk); d_skip (heads);
 *             psi, zeta, phi (heads, rank, dv); out HEAD-MAJOR (batch, heads, len, dv);
 *             last_state (batch, heads, dv, dqk); last_bx (batch, heads, dqk)
 */
#ifndef ARM_SCAN_HIP_H
#define ARM_SCAN_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ARM_SCAN_ABI_VERSION 9u

/* Return codes: arm-scan-ffi/src/lib.rs:53-58, plus 6. */
#define ARM_SCAN_OK 0
#define ARM_SCAN_ERR_NULL_POINTER 1
#define ARM_SCAN_ERR_INVALID_DIMS 2
#define ARM_SCAN_ERR_BACKEND_UNAVAILABLE 3
#define ARM_SCAN_ERR_BAD_ENUM 4
#define ARM_SCAN_ERR_PANIC 5
#define ARM_SCAN_ERR_DEVICE 6

/* backend: 0 auto (= the HIP kernels); 1 scalar and 2 neon are CPU backends of the
 * reference and return ARM_SCAN_ERR_BACKEND_UNAVAILABLE here.
 * threading: 0 auto, 1 sequential, 2 rayon — accepted for compatibility and ignored
 * (the GPU grid replaces Rayon); any other value is ARM_SCAN_ERR_BAD_ENUM. */

/* arm-scan-ffi/src/lib.rs:43-50, unchanged. */
typedef struct ArmScanDims {
  size_t batch, dim, len, state, groups;
} ArmScanDims;

/* arm-scan-ffi/src/lib.rs:362-373 plus `groups` (ABI 9). */
typedef struct ArmMamba3Dims {
  size_t batch, heads, dv, dqk, len, rank, groups;
} ArmMamba3Dims;

/* New in ABI 9: the 2D cross-scan over a (height, width) token grid. */
typedef struct ArmSS2DDims {
  size_t batch, dim, height, width, state;
} ArmSS2DDims;

/* Replaces arm_scan_abi_version (arm-scan-ffi/src/lib.rs:37-40); returns 9. */
uint32_t arm_scan_abi_version(void);

/* Replaces arm_scan_selective_scan_f32 (arm-scan-ffi/src/lib.rs:99-216).
 * Nullable: d_skip, z, delta_bias, last_state, h0. `reverse` walks the sequence
 * backward (output t still lands at index t; last_state is then the state after
 * consuming t == 0). h0 seeds the recurrence (orthogonal to reverse).
 * Device scratch, from a memory pool the library owns: the segment maps of the plan
 * for few rows and, for rows that are not 16-byte multiples (len % 4 != 0 or an
 * unaligned B/C), a copy of B and C at a padded row pitch. */
int arm_scan_selective_scan_f32(const ArmScanDims* dims, const float* u, const float* delta,
                                const float* a, const float* b, const float* c,
                                const float* d_skip, const float* z, const float* delta_bias,
                                int delta_softplus, int reverse, int backend, int threading,
                                float* out, float* last_state, const float* h0, void* stream);

/* No reference counterpart: arm_scan_selective_scan_f32 for callers that cannot
 * allocate device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same arguments, checks, codes and results (bit-identical); it
 * calls no hipMalloc/hipFree. Rows that are not 16-byte multiples read B and C in place
 * as single floats instead of through a padded copy. The only scratch it keeps, the
 * segment maps of the plan for few rows (B * D < 8192: rows cut into segments folded
 * first, then replayed), lives in a static 4 MiB device array, one per GPU, held until
 * the process ends.
 * No size is rejected for it: a plan whose maps would exceed 4 MiB is cut to fewer
 * segments (whole rows need none). Every map is written before it is read, so no
 * call depends on what the array held before. Calls on two streams of one GPU share
 * the array: a call made on a stream other than the previous call's makes its stream
 * wait for that call's kernels (an event, created at the first call on the GPU), so
 * they run one after the other. Calls recorded into a HIP graph are not ordered so:
 * the graph's dependencies must order them, or they race. */
int arm_scan_selective_scan_noalloc_f32(const ArmScanDims* dims, const float* u,
                                        const float* delta, const float* a, const float* b,
                                        const float* c, const float* d_skip, const float* z,
                                        const float* delta_bias, int delta_softplus,
                                        int reverse, int backend, int threading, float* out,
                                        float* last_state, const float* h0, void* stream);

/* No reference counterpart: arm_scan_selective_scan_f32 with u, z and out given by
 * element strides (batch, dim, step) instead of as contiguous (batch, dim, len).
 * It serves the Hugging Face seam, which hands the gate z as a (batch, dim, len)
 * view of time-major (batch, len, 2*dim) storage (transformers modeling_mamba.py
 * MambaMixer.forward -> mamba_selective_scan(..., z=gate)); the reference copies it
 * (python/arm_scan/op.py:19-20). Writing out time-major likewise lets the caller's
 * out_proj read it without a copy, and u may be a time-major view too (the mixer's
 * convolution output laid out for its x_proj). A null stride array means contiguous.
 * Needs len % 4 == 0, dim and dim/groups multiples of 16, 16-byte aligned delta/B/C
 * (and u when contiguous) and each batch of u/z/out inside 4 GiB; otherwise
 * ARM_SCAN_ERR_INVALID_DIMS, and the caller makes them contiguous and calls
 * arm_scan_selective_scan_f32. */
int arm_scan_selective_scan_strided_f32(const ArmScanDims* dims, const float* u,
                                        const long long* u_strides,
                                        const float* delta, const float* a, const float* b,
                                        const float* c, const float* d_skip, const float* z,
                                        const long long* z_strides, const float* delta_bias,
                                        int delta_softplus, int reverse, float* out,
                                        const long long* out_strides, float* last_state,
                                        const float* h0, void* stream);

/* No reference counterpart (the reference leaves decoding to upstream,
 * README.md:320-322): one step of the Mamba-1 scan for a generation loop, as
 * transformers' mamba_selective_state_update computes it, in one launch. state
 * (batch, dim, state_dim) is read and rewritten in place; x, dt, z are (batch, dim)
 * and B, C (batch, state_dim), each by element strides (null: contiguous); a
 * (dim, state_dim); out (batch, dim). dt_bias/dt_softplus as for the scan; d_skip, z
 * and dt_bias nullable. */
int arm_scan_selective_state_update_f32(
    size_t batch, size_t dim, size_t state_dim, float* state, const float* x,
    const long long* x_strides, const float* dt, const long long* dt_strides, const float* a,
    const float* b, const long long* b_strides, const float* c, const long long* c_strides,
    const float* d_skip, const float* z, const long long* z_strides, const float* dt_bias,
    int dt_softplus, float* out, void* stream);

/* Replaces arm_scan_selective_scan_bidirectional_f32 (arm-scan-ffi/src/lib.rs:235-354):
 * the forward and the reverse scan of the same inputs, both seeded from zero. Where its
 * 16-row blocks fill the chip the two directions are two traversals of one launch (each
 * evaluating exp(delta*A)); fewer rows that fit one on-chip pass share exp(delta*A) in
 * one kernel; other shapes run two launches.
 * last_fwd / last_bwd: both or neither (else ARM_SCAN_ERR_INVALID_DIMS). */
int arm_scan_selective_scan_bidirectional_f32(
    const ArmScanDims* dims, const float* u, const float* delta, const float* a,
    const float* b, const float* c, const float* d_skip, const float* z,
    const float* delta_bias, int delta_softplus, int backend, int threading, float* out_fwd,
    float* out_bwd, float* last_fwd, float* last_bwd, void* stream);

/* Replaces arm_scan_mamba3_scan_f32 (arm-scan-ffi/src/lib.rs:419-577).
 * psi/zeta/phi: all three (MIMO) or none (SISO), else ARM_SCAN_ERR_NULL_POINTER.
 * SISO: last_state/last_bx both or neither (else code 1). MIMO: last_state allowed,
 * last_bx rejected (code 2). trap is pre-sigmoid; cos/sin come from the angle
 * pre-pass; out is head-major. */
int arm_scan_mamba3_scan_f32(const ArmMamba3Dims* dims, const float* q, const float* k,
                             const float* v, const float* adt, const float* dt,
                             const float* trap, const float* q_bias, const float* k_bias,
                             const float* cos, const float* sin, const float* d_skip,
                             const float* z, const float* mimo_psi, const float* mimo_zeta,
                             const float* mimo_phi, int reverse, int backend, int threading,
                             float* out, float* last_state, float* last_bx, void* stream);

/* New in ABI 9 (no counterpart in the reference): arm_scan_mamba3_scan_f32 with out
 * written time-major (batch, len, heads, dv), the layout python/arm_scan/mamba3.py:142
 * produces from the head-major result with a permute and a copy. Same arguments,
 * checks and codes. */
int arm_scan_mamba3_scan_time_major_f32(
    const ArmMamba3Dims* dims, const float* q, const float* k, const float* v, const float* adt,
    const float* dt, const float* trap, const float* q_bias, const float* k_bias,
    const float* cos, const float* sin, const float* d_skip, const float* z,
    const float* mimo_psi, const float* mimo_zeta, const float* mimo_phi, int reverse,
    int backend, int threading, float* out, float* last_state, float* last_bx, void* stream);

/* No reference counterpart: arm_scan_mamba3_scan_time_major_f32 (forward) with the
 * angle pre-pass fused into the scan. The reference computes cos/sin in Python
 * (python/arm_scan/mamba3.py:41-89, theta = cumsum_l(tanh(angle) * pi * dt)) and
 * passes them in; here raw `angles` (b, l, h, n_angles) replace cos and sin, the
 * pairs past n_angles rotating by zero as in its padding. Needs n_angles a positive
 * multiple of 4 up to dqk/2, 16-byte aligned inputs and the chunked kernel's shapes
 * (dv, dqk multiples of 16, dqk <= 128, rank 1/2/4); otherwise
 * ARM_SCAN_ERR_INVALID_DIMS and the caller runs the pre-pass and calls
 * arm_scan_mamba3_scan_time_major_f32. There is no reverse: theta is a forward
 * cumsum, which a backward walk does not have. */
int arm_scan_mamba3_scan_angles_f32(
    const ArmMamba3Dims* dims, const float* q, const float* k, const float* v, const float* adt,
    const float* dt, const float* trap, const float* q_bias, const float* k_bias,
    const float* angles, size_t n_angles, const float* d_skip, const float* z,
    const float* mimo_psi, const float* mimo_zeta, const float* mimo_phi, int backend,
    int threading, float* out, float* last_state, float* last_bx, void* stream);

/* No reference counterpart: the forward Mamba-3 scan from raw angles with v, z and the
 * angles given by element strides, as the Mamba-3 mixer holds them: views into its
 * in_proj output, the angles shared by every head (apps/mamba3_lm/block.py:150-174
 * splits the projection, `expand`s the angles over heads, and the reference's
 * python/arm_scan/mamba3.py then copies each one contiguous).
 *   v_strides, z_strides: (batch, step) in elements; within a step the heads lie dv
 *     apart. angle_strides: (batch, step, head); the head stride may be 0.
 * Other arguments as arm_scan_mamba3_scan_angles_f32; out is time-major (b, l, h, dv)
 * and contiguous. Where the fused SISO kernel does not apply (MIMO, n_angles not a
 * multiple of 4, strides that are not multiples of 4), the angle pre-pass runs into
 * stream-ordered scratch and the scan reads cos/sin from it. The strides must keep
 * every access inside the caller's buffers; negative strides return
 * ARM_SCAN_ERR_INVALID_DIMS. */
int arm_scan_mamba3_scan_strided_f32(
    const ArmMamba3Dims* dims, const float* q, const float* k, const float* v,
    const int64_t* v_strides, const float* adt, const float* dt, const float* trap,
    const float* q_bias, const float* k_bias, const float* angles, size_t n_angles,
    const int64_t* angle_strides, const float* d_skip, const float* z, const int64_t* z_strides,
    const float* mimo_psi, const float* mimo_zeta, const float* mimo_phi, int backend,
    int threading, float* out, void* stream);

/* No reference counterpart: the Mamba-1 mixer's depthwise causal convolution, the step
 * before the scan in Hugging Face's MambaMixer (transformers modeling_mamba.py
 * causal_conv1d_fn), which the reference leaves to upstream (its patch replaces only
 * the scan, python/arm_scan/patch.py:119-180):
 *   out[b, d, t] = act(bias[d] + sum_{k < width} weight[d, k] x[b, d, t - width + 1 + k])
 * with x[t < 0] = 0 and act silu (silu = 1) or the identity (silu = 0). x is any strided
 * (batch, dim, len) view given by x_strides (batch, dim, step) in elements; the mixer
 * passes the time-major half of its in_proj output. weight (dim, width), bias (dim) or
 * NULL; out (batch, dim, len) contiguous, or with out_time_major = 1 (batch, len, dim)
 * storage, the layout the mixer's x_proj reads. width <= 8. */
int arm_scan_causal_conv1d_f32(size_t batch, size_t dim, size_t len, size_t width,
                               const float* x, const int64_t* x_strides, const float* weight,
                               const float* bias, int silu, int out_time_major, float* out,
                               void* stream);

/* No reference counterpart: one decode step of arm_scan_causal_conv1d_f32, transformers'
 * causal_conv1d_update: conv_state (batch, dim, width) contiguous holds the last width
 * inputs; it is shifted left in place with x (batch, dim; strides x_strides) appended,
 * and out (batch, dim) = act(bias + sum_k weight[d, k] conv_state[b, d, k]) after the
 * shift. width <= 64. */
int arm_scan_causal_conv1d_update_f32(size_t batch, size_t dim, size_t width,
                                      const float* x, const int64_t* x_strides,
                                      float* conv_state, const float* weight,
                                      const float* bias, int silu, float* out, void* stream);

/* No reference counterpart: the Mamba-3 mixer's front-end, which the reference runs as
 * torch ops (apps/mamba3_lm/block.py:146-178), in one kernel. proj (batch, len,
 * row_stride) is the in_proj output with the checkpoint's column order
 * [z (h*headdim) | x (h*headdim) | B (r*g*d_state) | C (r*g*d_state) | dd_dt (h) |
 * dd_A (h) | trap (h) | angles (n_angles)] (block.py:113-118). Writes
 *   dt = softplus(dd_dt + dt_bias), adt = min(-heavy_tail(dd_A), -a_floor) * dt and
 *   trap, each (batch, heads, len);
 *   k = RMSNorm(B) * b_norm_weight and q = RMSNorm(C) * c_norm_weight, each (batch,
 *   len, rank, groups, d_state), eps inside the square root (Q <- C, K <- B).
 * z, x and the angles are left where they are, for arm_scan_mamba3_scan_strided_f32. */
int arm_scan_mamba3_block_frontend_f32(
    const float* proj, size_t batch, size_t len, size_t row_stride, size_t heads,
    size_t headdim, size_t d_state, size_t rank, size_t groups, size_t n_angles,
    const float* dt_bias, float a_floor, const float* b_norm_weight, const float* c_norm_weight,
    float norm_eps, float* q, float* k, float* adt, float* dt, float* trap, void* stream);

/* No reference counterpart: the non-causal Mamba-3 SISO aggregation, which the
 * reference composes in Python over its two traversals (python/arm_scan/
 * mamba3_noncausal.py:89-98: forward + backward - the same-step term counted twice).
 * Arguments are arm_scan_mamba3_scan_f32's for rank 1 without the MIMO projections,
 * carries or direction; out is written TIME-MAJOR (batch, len, heads, dv). The
 * forward traversal writes out; the backward one leaves the same-step term
 * (gamma q.k + D) out and adds onto it, so no second output and no diagonal pass
 * exist. ARM_SCAN_ERR_INVALID_DIMS for rank != 1. */
int arm_scan_mamba3_noncausal_f32(const ArmMamba3Dims* dims, const float* q, const float* k,
                                  const float* v, const float* adt, const float* dt,
                                  const float* trap, const float* q_bias, const float* k_bias,
                                  const float* cos, const float* sin, const float* d_skip,
                                  const float* z, int backend, int threading, float* out,
                                  void* stream);

/* No reference counterpart: the RoPE angle pre-pass the reference runs in Python
 * (python/arm_scan/mamba3.py:41-89), as two kernels (the sums of sequence segments,
 * then cos/sin from them). angles (batch, len, heads, n_angles) raw, dt (batch, heads,
 * len) post-softplus -> cos, sin (batch, len, heads, half) with
 * theta = cumsum_len(tanh(angle) * pi * dt); pairs n_angles .. half-1 get cos 1,
 * sin 0. Feeds arm_scan_mamba3_scan[_time_major]_f32 where the fused entry point does
 * not apply (reverse, MIMO, n_angles not a multiple of 4). */
int arm_scan_mamba3_angles_f32(const float* angles, const float* dt, size_t batch, size_t len,
                               size_t heads, size_t n_angles, size_t half, float* cos,
                               float* sin, void* stream);

/* New in ABI 9 (no single reference symbol: it fuses python/arm_scan/ss2d.py:277-342,
 * which composes two bidirectional calls). Four directions over a (H, W) grid:
 * row_fwd, row_bwd over the row-major flattening t = i*W + j, col_fwd, col_bwd over the
 * column-major one t = j*H + i; backward = reverse index mode.
 *   u, delta, z, out-planes (batch, dim, H, W); a (dim, state); d_skip, delta_bias (dim);
 *   b4, c4 (4, batch, state, H, W): one B and one C per direction, in grid layout
 *   (the token at (i, j) uses b4[k][.., i, j] in direction k).
 * merge: 0 none -> out is (4, batch, dim, H, W), the planes in the order above;
 *        1 sum  -> out is (batch, dim, H, W) = sum of the planes; 2 mean -> sum / 4.
 * D and z apply inside every direction (a sum carries 4*D*u), as in the reference.
 * last_states (4, batch, dim, state) is nullable. */
int arm_scan_ss2d_f32(const ArmSS2DDims* dims, const float* u, const float* delta,
                      const float* a, const float* b4, const float* c4, const float* d_skip,
                      const float* z, const float* delta_bias, int delta_softplus, int merge,
                      float* out, float* last_states, void* stream);

/* Human-readable reason for the last nonzero code returned on this thread. */
const char* arm_scan_last_error(void);

#ifdef __cplusplus
}
#endif

#endif /* ARM_SCAN_HIP_H */
