// C ABI of libarm_scan_hip.so (declared in include/arm_scan_hip.h).
//
// Host-side validation follows the reference's FFI layer
// (kernel/arm-scan-ffi/src/lib.rs:99-577) and its core checks
// (arm-scan-core/src/lib.rs:181-249, mamba3/mod.rs:213-335): null pointers -> 1,
// bad enums -> 4, zero / overflowing / non-dividing dims -> 2, unavailable
// backend -> 3, all before any launch. Code 6 reports a HIP error.

#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdarg>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>

#include "../../include/arm_scan_hip.h"
#include "scan_launch.h"

namespace {

thread_local std::string g_last_error;

int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
int fail(int code, const char* fmt, ...) {
  char buf[512];
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(buf, sizeof(buf), fmt, ap);
  va_end(ap);
  g_last_error = buf;
  return code;
}

int hip_fail(hipError_t e, const char* where) {
  return fail(ARM_SCAN_ERR_DEVICE, "%s: %s", where, hipGetErrorString(e));
}

bool mul_ok(size_t a, size_t b, size_t* out) { return !__builtin_mul_overflow(a, b, out); }
bool prod_ok(std::initializer_list<size_t> xs) {
  size_t acc = 1;
  for (size_t x : xs)
    if (!mul_ok(acc, x, &acc)) return false;
  return true;
}

// backend 0 = auto (the HIP kernels); 1 scalar / 2 neon are CPU backends of the
// reference. threading is accepted and ignored.
int check_enums(int backend, int threading) {
  if (backend < 0 || backend > 2 || threading < 0 || threading > 2)
    return fail(ARM_SCAN_ERR_BAD_ENUM, "bad backend (%d) or threading (%d) enum", backend,
                threading);
  if (backend != 0)
    return fail(ARM_SCAN_ERR_BACKEND_UNAVAILABLE,
                "backend %d is a CPU backend; this library runs backend 0 (HIP)", backend);
  return ARM_SCAN_OK;
}

int check_m1_dims(const ArmScanDims& d) {
  if (!prod_ok({d.batch, d.dim, d.len}) || !prod_ok({d.batch, d.groups, d.state, d.len}) ||
      !prod_ok({d.dim, d.state}) || !prod_ok({d.batch, d.dim, d.state}))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "dims overflow size_t");
  if (!d.batch || !d.dim || !d.len || !d.state || !d.groups)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "a dimension is zero");
  if (d.dim % d.groups)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "groups (%zu) does not divide dim (%zu)", d.groups,
                d.dim);
  // device-side index arithmetic uses 32-bit row counts and 64-bit offsets
  if (d.batch * d.dim > (1u << 30) || d.len > (1ull << 40))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "problem too large for this build");
  return ARM_SCAN_OK;
}

int run(hipError_t e, const char* where) {
  if (e != hipSuccess) return hip_fail(e, where);
  return ARM_SCAN_OK;
}

// The allocation-free entry's calls share one static scratch array per device. A call
// on a stream other than the previous call's first makes its stream wait for an event
// recorded after that call's kernels, so calls made on two streams run one after the
// other instead of racing on the array. The event is created once per device, at the
// first call there. A stream being captured into a graph is left alone (an event from
// outside the capture cannot order it), and so is the order of the captured calls:
// the graph's own dependencies must order them.
class ScratchOrder {
 public:
  // Before the call's launches: order `st` after the previous call, if on another stream.
  hipError_t enter(hipStream_t st) {
    mu_.lock();
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    hipError_t e = hipStreamIsCapturing(st, &cs);
    if (e != hipSuccess) {  // a query refused during another stream's capture: order nothing
      (void)hipGetLastError();
      cs = hipStreamCaptureStatusActive;
      e = hipSuccess;
    }
    capturing_ = cs != hipStreamCaptureStatusNone;
    if (!capturing_) {
      if (done_ == nullptr) e = hipEventCreateWithFlags(&done_, hipEventDisableTiming);
      if (e == hipSuccess && used_ && last_ != st) e = hipStreamWaitEvent(st, done_, 0);
    }
    if (e != hipSuccess) mu_.unlock();
    return e;
  }
  // After them (only after a successful enter): mark the call's end on its stream.
  hipError_t leave(hipStream_t st, bool launched) {
    hipError_t e = hipSuccess;
    if (launched && !capturing_) {
      e = hipEventRecord(done_, st);
      used_ = e == hipSuccess;
      last_ = st;
    }
    mu_.unlock();
    return e;
  }

 private:
  std::mutex mu_;
  hipEvent_t done_ = nullptr;
  hipStream_t last_ = nullptr;
  bool used_ = false, capturing_ = false;
};

ScratchOrder* scratch_order() {
  constexpr int kMaxDevices = 64;
  static ScratchOrder orders[kMaxDevices];
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return nullptr;
  return &orders[dev];
}

}  // namespace

namespace armscan {

// Per-call scratch (gate records, SS2D planes, segment maps, cos/sin) comes from a
// memory pool the library owns, one per device, created on first use and kept until
// the process ends. Its release threshold keeps freed blocks for the next call, so a
// steady stream of calls allocates from memory already mapped; the device's default
// pool, which the caller or torch may use, keeps its own settings. Where a pool cannot
// be created, the scratch comes from the default pool as it is.
hipError_t stream_alloc(void** p, size_t bytes, hipStream_t st) {
  constexpr int kMaxDevices = 64;
  static std::atomic<hipMemPool_t> pools[kMaxDevices] = {};
  static std::atomic<bool> no_pool[kMaxDevices] = {};
  static std::mutex create_mu;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= kMaxDevices) return hipErrorInvalidDevice;
  hipMemPool_t pool = pools[dev].load(std::memory_order_acquire);
  if (pool == nullptr && !no_pool[dev].load(std::memory_order_acquire)) {
    std::lock_guard<std::mutex> lock(create_mu);
    pool = pools[dev].load(std::memory_order_acquire);
    if (pool == nullptr && !no_pool[dev].load(std::memory_order_relaxed)) {
      hipMemPoolProps props{};
      props.allocType = hipMemAllocationTypePinned;
      props.handleTypes = hipMemHandleTypeNone;
      props.location.type = hipMemLocationTypeDevice;
      props.location.id = dev;
      uint64_t keep = UINT64_MAX;
      if (hipMemPoolCreate(&pool, &props) != hipSuccess) {
        pool = nullptr;
        (void)hipGetLastError();  // the failed creation leaves no error behind
      } else if (hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep) !=
                 hipSuccess) {
        (void)hipMemPoolDestroy(pool);
        pool = nullptr;
        (void)hipGetLastError();
      }
      if (pool != nullptr) pools[dev].store(pool, std::memory_order_release);
      else no_pool[dev].store(true, std::memory_order_release);
    }
  }
  if (pool == nullptr) return hipMallocAsync(p, bytes, st);
  return hipMallocFromPoolAsync(p, bytes, pool, st);
}

}  // namespace armscan

extern "C" {

uint32_t arm_scan_abi_version(void) { return ARM_SCAN_ABI_VERSION; }

const char* arm_scan_last_error(void) { return g_last_error.c_str(); }

int arm_scan_selective_scan_f32(const ArmScanDims* dims, const float* u, const float* delta,
                                const float* a, const float* b, const float* c,
                                const float* d_skip, const float* z, const float* delta_bias,
                                int delta_softplus, int reverse, int backend, int threading,
                                float* out, float* last_state, const float* h0, void* stream) {
  if (!dims || !u || !delta || !a || !b || !c || !out)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (int rc = check_enums(backend, threading)) return rc;
  if (int rc = check_m1_dims(*dims)) return rc;
  armscan::M1Problem p{};
  p.batch = dims->batch; p.dim = dims->dim; p.len = dims->len; p.state = dims->state;
  p.groups = dims->groups;
  p.u = u; p.delta = delta; p.A = a; p.B = b; p.C = c; p.D = d_skip; p.z = z;
  p.bias = delta_bias; p.h0 = h0; p.out = out; p.last = last_state;
  p.softplus = delta_softplus != 0; p.reverse = reverse != 0;
  return run(armscan::m1_scan(p, (hipStream_t)stream), "selective_scan launch");
}

int arm_scan_selective_scan_noalloc_f32(const ArmScanDims* dims, const float* u,
                                        const float* delta, const float* a, const float* b,
                                        const float* c, const float* d_skip, const float* z,
                                        const float* delta_bias, int delta_softplus,
                                        int reverse, int backend, int threading, float* out,
                                        float* last_state, const float* h0, void* stream) {
  if (!dims || !u || !delta || !a || !b || !c || !out)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (int rc = check_enums(backend, threading)) return rc;
  if (int rc = check_m1_dims(*dims)) return rc;
  armscan::M1Problem p{};
  p.batch = dims->batch; p.dim = dims->dim; p.len = dims->len; p.state = dims->state;
  p.groups = dims->groups;
  p.u = u; p.delta = delta; p.A = a; p.B = b; p.C = c; p.D = d_skip; p.z = z;
  p.bias = delta_bias; p.h0 = h0; p.out = out; p.last = last_state;
  p.softplus = delta_softplus != 0; p.reverse = reverse != 0;
  // the segment maps go to the library's static scratch on this device: nothing is
  // allocated, and the plan never needs more than the scratch holds
  if (hipError_t e = armscan::m1_noalloc_scratch(&p.scratch, &p.scratch_bytes))
    return hip_fail(e, "scratch lookup");
  const hipStream_t st = (hipStream_t)stream;
  ScratchOrder* order = scratch_order();
  if (order == nullptr) return hip_fail(hipErrorInvalidDevice, "scratch order");
  if (hipError_t e = order->enter(st)) return hip_fail(e, "ordering after the previous call");
  const hipError_t e = armscan::m1_scan(p, st);
  const hipError_t e2 = order->leave(st, e == hipSuccess);
  if (e != hipSuccess) return hip_fail(e, "selective_scan (no-alloc) launch");
  return run(e2, "recording the call's end");
}

int arm_scan_selective_scan_strided_f32(const ArmScanDims* dims, const float* u,
                                        const long long* u_strides,
                                        const float* delta, const float* a, const float* b,
                                        const float* c, const float* d_skip, const float* z,
                                        const long long* z_strides, const float* delta_bias,
                                        int delta_softplus, int reverse, float* out,
                                        const long long* out_strides, float* last_state,
                                        const float* h0, void* stream) {
  if (!dims || !u || !delta || !a || !b || !c || !out)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (int rc = check_m1_dims(*dims)) return rc;
  armscan::M1Problem p{};
  p.batch = dims->batch; p.dim = dims->dim; p.len = dims->len; p.state = dims->state;
  p.groups = dims->groups;
  p.u = u; p.delta = delta; p.A = a; p.B = b; p.C = c; p.D = d_skip; p.z = z;
  p.bias = delta_bias; p.h0 = h0; p.out = out; p.last = last_state;
  p.softplus = delta_softplus != 0; p.reverse = reverse != 0;
  // a null stride array is the contiguous (batch, dim, len) layout; given strides are
  // taken as they are (a 0 is a broadcast view, read in place)
  const long long cont[3] = {(long long)(dims->dim * dims->len), (long long)dims->len, 1};
  p.has_strides = 1;
  for (int i = 0; i < 3; ++i) {
    p.z_stride[i] = z_strides ? z_strides[i] : cont[i];
    p.out_stride[i] = out_strides ? out_strides[i] : cont[i];
    p.u_stride[i] = u_strides ? u_strides[i] : cont[i];
  }
  const char* why = nullptr;
  if (armscan::m1_strided_io(p) && !armscan::m1_strided_supported(p, &why))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "%s", why);
  return run(armscan::m1_scan(p, (hipStream_t)stream), "selective_scan (strided) launch");
}

int arm_scan_selective_state_update_f32(
    size_t batch, size_t dim, size_t state_dim, float* state, const float* x,
    const long long* x_strides, const float* dt, const long long* dt_strides, const float* a,
    const float* b, const long long* b_strides, const float* c, const long long* c_strides,
    const float* d_skip, const float* z, const long long* z_strides, const float* dt_bias,
    int dt_softplus, float* out, void* stream) {
  if (!state || !x || !dt || !a || !b || !c || !out)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (!batch || !dim || !state_dim) return fail(ARM_SCAN_ERR_INVALID_DIMS, "a dimension is zero");
  if (!prod_ok({batch, dim, state_dim}) || batch * dim > (1u << 30) || state_dim > (1u << 20))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "problem too large for this build");
  armscan::M1Step p{};
  p.state = state; p.x = x; p.dt = dt; p.A = a; p.B = b; p.C = c; p.D = d_skip; p.z = z;
  p.bias = dt_bias; p.out = out;
  p.batch = (int)batch; p.dim = (int)dim; p.N = (int)state_dim; p.softplus = dt_softplus != 0;
  auto st2 = [](long long* dst, const long long* src, long long s0, long long s1) {
    dst[0] = src ? src[0] : s0;
    dst[1] = src ? src[1] : s1;
    return dst[0] >= 0 && dst[1] >= 0;
  };
  const long long D = (long long)dim, N = (long long)state_dim;
  if (!st2(p.xs, x_strides, D, 1) || !st2(p.dts, dt_strides, D, 1) ||
      !st2(p.zs, z_strides, D, 1) || !st2(p.Bs, b_strides, N, 1) ||
      !st2(p.Cs, c_strides, N, 1))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "negative strides");
  return run(armscan::m1_step(p, (hipStream_t)stream), "state update launch");
}

int arm_scan_selective_scan_bidirectional_f32(
    const ArmScanDims* dims, const float* u, const float* delta, const float* a,
    const float* b, const float* c, const float* d_skip, const float* z,
    const float* delta_bias, int delta_softplus, int backend, int threading, float* out_fwd,
    float* out_bwd, float* last_fwd, float* last_bwd, void* stream) {
  if (!dims || !u || !delta || !a || !b || !c || !out_fwd || !out_bwd)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (int rc = check_enums(backend, threading)) return rc;
  if (int rc = check_m1_dims(*dims)) return rc;
  if ((last_fwd == nullptr) != (last_bwd == nullptr))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "last_fwd and last_bwd must both be set or null");
  armscan::M1Problem p{};
  p.batch = dims->batch; p.dim = dims->dim; p.len = dims->len; p.state = dims->state;
  p.groups = dims->groups;
  p.u = u; p.delta = delta; p.A = a; p.B = b; p.C = c; p.D = d_skip; p.z = z;
  p.bias = delta_bias; p.softplus = delta_softplus != 0;
  hipStream_t st = (hipStream_t)stream;
  // Both directions as two traversals of one launch of the streaming chunk kernel: it
  // evaluates exp(dt A) once per direction, yet at B16 D192 it takes 49 / 91 / 173 us
  // for L 1024 / 2048 / 4096 against 59 / 92 us for the single-pass kernel that shares
  // the exp (whose whole-row scans and barriers cost more than the exp they save) and
  // 222 us for two launches at L 4096. That launch scans whole rows, one 16-row block
  // per direction, so it is taken where those blocks give every CU one (B16 D192: 384
  // blocks), or where rows are too short to cut into segments anyway. Fewer rows take
  // the exp-sharing kernel where a row fits it (B1 D1536 L2048: 84 us against 114 us
  // for two segmented calls), else two launches, each cutting its rows into segments
  // (B1 D16 L65536: 174 us; B1 D768 L32768: 401 us).
  p.out = out_fwd;
  const bool jobs_fill = 2 * (dims->batch * dims->dim / 16) >= armscan::kM1JobsMinBlocks ||
                         dims->len < 2 * armscan::kM1ChunkSteps;
  if (jobs_fill && armscan::m1_jobs_supported(p)) {
    const armscan::M1JobSpec jobs[2] = {{u, delta, z, b, c, out_fwd, last_fwd, 0},
                                        {u, delta, z, b, c, out_bwd, last_bwd, 1}};
    return run(armscan::m1_scan_jobs(p, jobs, 2, st), "bidirectional launch");
  }
  if (armscan::m1_bidir_fusable(p)) {
    p.out = out_fwd; p.out2 = out_bwd; p.last = last_fwd; p.last2 = last_bwd;
    return run(armscan::m1_bidir(p, st), "bidirectional launch");
  }
  p.out = out_fwd; p.last = last_fwd; p.reverse = 0;
  if (int rc = run(armscan::m1_scan(p, st), "bidirectional (forward) launch")) return rc;
  p.out = out_bwd; p.last = last_bwd; p.reverse = 1;
  return run(armscan::m1_scan(p, st), "bidirectional (reverse) launch");
}

static int mamba3_call(const ArmMamba3Dims* dims, const float* q, const float* k,
                       const float* v, const float* adt, const float* dt, const float* trap,
                       const float* q_bias, const float* k_bias, const float* cos,
                       const float* sin, const float* d_skip, const float* z,
                       const float* mimo_psi, const float* mimo_zeta, const float* mimo_phi,
                       int reverse, int backend, int threading, float* out, float* last_state,
                       float* last_bx, void* stream, bool time_major,
                       const float* angles = nullptr, size_t n_angles = 0,
                       bool accumulate = false, const int64_t* v_strides = nullptr,
                       const int64_t* z_strides = nullptr,
                       const int64_t* angle_strides = nullptr, bool unfused_ok = false) {
  if (!dims || !q || !k || !v || !adt || !dt || !trap || !q_bias || !k_bias || !out ||
      (angles ? false : (!cos || !sin)))
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  const int n_mimo = (mimo_psi != nullptr) + (mimo_zeta != nullptr) + (mimo_phi != nullptr);
  const bool mimo = n_mimo == 3;
  if (n_mimo != 0 && n_mimo != 3)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "psi/zeta/phi must be all set or all null");
  if (!mimo && (last_state == nullptr) != (last_bx == nullptr))
    return fail(ARM_SCAN_ERR_NULL_POINTER, "last_state and last_bx must both be set or null");
  if (int rc = check_enums(backend, threading)) return rc;
  const ArmMamba3Dims& d = *dims;
  if (d.dqk % 2) return fail(ARM_SCAN_ERR_INVALID_DIMS, "dqk (%zu) must be even", d.dqk);
  if (!d.batch || !d.heads || !d.dv || !d.dqk || !d.len || !d.rank || !d.groups)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "a dimension is zero");
  if (!prod_ok({d.batch, d.len, d.rank, d.groups, d.dqk}) ||
      !prod_ok({d.batch, d.len, d.heads, d.dv}) || !prod_ok({d.batch, d.heads, d.dv, d.dqk}) ||
      !prod_ok({d.heads, d.rank, d.dqk}) || !prod_ok({d.heads, d.rank, d.dv}))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "dims overflow size_t");
  if (d.heads % d.groups)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "groups (%zu) does not divide heads (%zu)", d.groups,
                d.heads);
  if (d.rank > 1 && !mimo)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "rank > 1 requires the MIMO projections");
  if (mimo && last_bx)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "MIMO has no last_bx carry (rank > 1 k per step)");
  if (d.len > (1u << 30) || d.batch * d.heads > (1u << 30))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "problem too large for this build");
  armscan::M3Problem p{};
  p.batch = d.batch; p.heads = d.heads; p.dv = d.dv; p.dqk = d.dqk; p.len = d.len;
  p.rank = d.rank; p.groups = d.groups;
  p.q = q; p.k = k; p.v = v; p.adt = adt; p.dt = dt; p.trap = trap; p.q_bias = q_bias;
  p.k_bias = k_bias; p.cos = cos; p.sin = sin; p.D = d_skip; p.z = z;
  p.psi = mimo_psi; p.zeta = mimo_zeta; p.phi = mimo_phi;
  p.out = out; p.last_state = last_state; p.last_bx = last_bx; p.reverse = reverse != 0;
  p.out_time_major = time_major ? 1 : 0;
  p.angles = angles;
  p.n_angles = n_angles;
  p.accumulate = accumulate ? 1 : 0;
  if (accumulate && (mimo || d.rank != 1))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "the non-causal sum is SISO (rank 1)");
  armscan::m3_contiguous_strides(p);  // then the caller's strides, as given
  for (int i = 0; i < 3; ++i) {
    if ((i < 2 && v_strides && v_strides[i] < 0) || (i < 2 && z_strides && z_strides[i] < 0) ||
        (angle_strides && angle_strides[i] < 0))
      return fail(ARM_SCAN_ERR_INVALID_DIMS, "strides must be non-negative");
    if (i < 2 && v_strides) p.v_strides[i] = (long long)v_strides[i];
    if (i < 2 && z_strides) p.z_strides[i] = (long long)z_strides[i];
    if (angle_strides) p.ang_strides[i] = (long long)angle_strides[i];
  }
  if (angles) {
    if (!prod_ok({d.batch, d.len, d.heads, n_angles}))
      return fail(ARM_SCAN_ERR_INVALID_DIMS, "dims overflow size_t");
    if (n_angles == 0 || n_angles > d.dqk / 2)
      return fail(ARM_SCAN_ERR_INVALID_DIMS, "n_angles (%zu) must be 1 .. dqk/2", n_angles);
    const char* why = nullptr;
    // with the unfused route at hand, MIMO takes it: its 16/rank-step chunks make the
    // fused pre-pass lengthen every iteration of a latency-bound loop
    if (!armscan::m3_angles_supported(p, &why) || (unfused_ok && mimo)) {
      if (!unfused_ok) return fail(ARM_SCAN_ERR_INVALID_DIMS, "%s", why);
      // the pre-pass kernels into scratch cos/sin, then the scan on them
      const size_t half = d.dqk / 2, n_cs = d.batch * d.len * d.heads * half;
      hipStream_t st = (hipStream_t)stream;
      float* cs = nullptr;
      hipError_t e = armscan::stream_alloc((void**)&cs, 2 * n_cs * sizeof(float), st);
      if (e != hipSuccess) return hip_fail(e, "angle scratch allocation");
      e = armscan::m3_angles_to_cos_sin(angles, dt, d.batch, d.len, d.heads, n_angles, half, cs,
                                        cs + n_cs, st, p.ang_strides);
      p.angles = nullptr;
      p.n_angles = 0;
      p.cos = cs;
      p.sin = cs + n_cs;
      if (e == hipSuccess) e = armscan::m3_scan(p, st);
      const hipError_t ef = hipFreeAsync(cs, st);
      return run(e != hipSuccess ? e : ef, "mamba3 (angle pre-pass, then scan) launch");
    }
  }
  // the chunked MFMA kernel takes dv, dqk multiples of 16 (dqk <= 128) and rank 1/2/4;
  // everything else runs the step-by-step kernel, whose state must fit in LDS
  const size_t need = d.dv * (d.dqk + 1) + 2 * d.rank * (d.dqk + d.dv) + d.rank * d.rank + 4;
  if (!armscan::m3_chunk_supported(p) && need > armscan::m3_max_state())
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "state dv*dqk (%zu x %zu) exceeds on-chip capacity",
                d.dv, d.dqk);
  return run(armscan::m3_scan(p, (hipStream_t)stream), "mamba3 launch");
}

int arm_scan_mamba3_scan_f32(const ArmMamba3Dims* dims, const float* q, const float* k,
                             const float* v, const float* adt, const float* dt,
                             const float* trap, const float* q_bias, const float* k_bias,
                             const float* cos, const float* sin, const float* d_skip,
                             const float* z, const float* mimo_psi, const float* mimo_zeta,
                             const float* mimo_phi, int reverse, int backend, int threading,
                             float* out, float* last_state, float* last_bx, void* stream) {
  return mamba3_call(dims, q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z,
                     mimo_psi, mimo_zeta, mimo_phi, reverse, backend, threading, out, last_state,
                     last_bx, stream, false);
}

int arm_scan_mamba3_scan_time_major_f32(
    const ArmMamba3Dims* dims, const float* q, const float* k, const float* v, const float* adt,
    const float* dt, const float* trap, const float* q_bias, const float* k_bias,
    const float* cos, const float* sin, const float* d_skip, const float* z,
    const float* mimo_psi, const float* mimo_zeta, const float* mimo_phi, int reverse,
    int backend, int threading, float* out, float* last_state, float* last_bx, void* stream) {
  return mamba3_call(dims, q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z,
                     mimo_psi, mimo_zeta, mimo_phi, reverse, backend, threading, out, last_state,
                     last_bx, stream, true);
}

int arm_scan_mamba3_scan_angles_f32(
    const ArmMamba3Dims* dims, const float* q, const float* k, const float* v, const float* adt,
    const float* dt, const float* trap, const float* q_bias, const float* k_bias,
    const float* angles, size_t n_angles, const float* d_skip, const float* z,
    const float* mimo_psi, const float* mimo_zeta, const float* mimo_phi, int backend,
    int threading, float* out, float* last_state, float* last_bx, void* stream) {
  if (!angles) return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  return mamba3_call(dims, q, k, v, adt, dt, trap, q_bias, k_bias, nullptr, nullptr, d_skip, z,
                     mimo_psi, mimo_zeta, mimo_phi, 0, backend, threading, out, last_state,
                     last_bx, stream, true, angles, n_angles);
}

int arm_scan_mamba3_scan_strided_f32(
    const ArmMamba3Dims* dims, const float* q, const float* k, const float* v,
    const int64_t* v_strides, const float* adt, const float* dt, const float* trap,
    const float* q_bias, const float* k_bias, const float* angles, size_t n_angles,
    const int64_t* angle_strides, const float* d_skip, const float* z, const int64_t* z_strides,
    const float* mimo_psi, const float* mimo_zeta, const float* mimo_phi, int backend,
    int threading, float* out, void* stream) {
  if (!angles || !v_strides || !angle_strides || (z && !z_strides))
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  return mamba3_call(dims, q, k, v, adt, dt, trap, q_bias, k_bias, nullptr, nullptr, d_skip, z,
                     mimo_psi, mimo_zeta, mimo_phi, 0, backend, threading, out, nullptr,
                     nullptr, stream, true, angles, n_angles, false, v_strides,
                     z ? z_strides : nullptr, angle_strides, true);
}

int arm_scan_causal_conv1d_f32(size_t batch, size_t dim, size_t len, size_t width,
                               const float* x, const int64_t* x_strides, const float* weight,
                               const float* bias, int silu, int out_time_major, float* out,
                               void* stream) {
  if (!x || !x_strides || !weight || !out)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (!batch || !dim || !len || !width)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "a dimension is zero");
  if (width > 8) return fail(ARM_SCAN_ERR_INVALID_DIMS, "width (%zu) above 8", width);
  if (batch > 65535 || dim > (1u << 22) || len > (1ull << 40) || !prod_ok({batch, dim, len}))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "problem too large for this build");
  for (int i = 0; i < 3; ++i)
    if (x_strides[i] < 0) return fail(ARM_SCAN_ERR_INVALID_DIMS, "strides must be non-negative");
  if (silu != 0 && silu != 1) return fail(ARM_SCAN_ERR_BAD_ENUM, "silu must be 0 or 1");
  if (out_time_major != 0 && out_time_major != 1)
    return fail(ARM_SCAN_ERR_BAD_ENUM, "out_time_major must be 0 or 1");
  armscan::CausalConv c{};
  c.out_tm = out_time_major;
  c.x = x;
  for (int i = 0; i < 3; ++i) c.xs[i] = (long long)x_strides[i];
  c.w = weight; c.bias = bias; c.out = out;
  c.batch = (int)batch; c.dim = (int)dim; c.width = (int)width; c.silu = silu;
  c.len = (long long)len;
  return run(armscan::causal_conv1d(c, (hipStream_t)stream), "causal conv1d launch");
}

int arm_scan_causal_conv1d_update_f32(size_t batch, size_t dim, size_t width,
                                      const float* x, const int64_t* x_strides,
                                      float* conv_state, const float* weight,
                                      const float* bias, int silu, float* out, void* stream) {
  if (!x || !x_strides || !conv_state || !weight || !out)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (!batch || !dim || !width) return fail(ARM_SCAN_ERR_INVALID_DIMS, "a dimension is zero");
  if (width > 64 || batch > (1u << 30) || dim > (1u << 30) || !prod_ok({batch, dim, width}))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "problem too large for this build");
  if (x_strides[0] < 0 || x_strides[1] < 0)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "strides must be non-negative");
  if (silu != 0 && silu != 1) return fail(ARM_SCAN_ERR_BAD_ENUM, "silu must be 0 or 1");
  armscan::CausalConvStep c{};
  c.x = x; c.xs[0] = (long long)x_strides[0]; c.xs[1] = (long long)x_strides[1];
  c.state = conv_state; c.w = weight; c.bias = bias; c.out = out;
  c.batch = (int)batch; c.dim = (int)dim; c.width = (int)width; c.silu = silu;
  return run(armscan::causal_conv1d_step(c, (hipStream_t)stream), "causal conv1d step launch");
}

int arm_scan_mamba3_block_frontend_f32(
    const float* proj, size_t batch, size_t len, size_t row_stride, size_t heads,
    size_t headdim, size_t d_state, size_t rank, size_t groups, size_t n_angles,
    const float* dt_bias, float a_floor, const float* b_norm_weight, const float* c_norm_weight,
    float norm_eps, float* q, float* k, float* adt, float* dt, float* trap, void* stream) {
  if (!proj || !dt_bias || !b_norm_weight || !c_norm_weight || !q || !k || !adt || !dt ||
      !trap)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (!batch || !len || !heads || !headdim || !d_state || !rank || !groups)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "a dimension is zero");
  if (heads % groups)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "groups (%zu) does not divide heads (%zu)", groups,
                heads);
  if (batch > 65535 || len > (1u << 30) || heads > 4096 || d_state > (1u << 20) ||
      rank * groups > 4096 || headdim > (1u << 20))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "problem too large for this build");
  const size_t need = 2 * heads * headdim + 2 * rank * groups * d_state + 3 * heads + n_angles;
  if (row_stride < need)
    return fail(ARM_SCAN_ERR_INVALID_DIMS,
                "row_stride (%zu) is shorter than the projection's columns (%zu)", row_stride,
                need);
  if (!prod_ok({batch, len, row_stride}) || !prod_ok({batch, len, rank, groups, d_state}))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "dims overflow size_t");
  if (!(norm_eps >= 0.0f) || !(a_floor == a_floor))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "norm_eps must be >= 0 and a_floor a number");
  armscan::M3Frontend f{};
  f.proj = proj; f.row_stride = (long long)row_stride;
  f.batch = (int)batch; f.len = (int)len; f.heads = (int)heads; f.headdim = (int)headdim;
  f.d_state = (int)d_state; f.rank = (int)rank; f.groups = (int)groups;
  f.dt_bias = dt_bias; f.b_norm = b_norm_weight; f.c_norm = c_norm_weight;
  f.a_floor = a_floor; f.eps = norm_eps;
  f.q = q; f.k = k; f.adt = adt; f.dt = dt; f.trap = trap;
  return run(armscan::m3_frontend(f, (hipStream_t)stream), "mamba3 front-end launch");
}

int arm_scan_mamba3_noncausal_f32(const ArmMamba3Dims* dims, const float* q, const float* k,
                                  const float* v, const float* adt, const float* dt,
                                  const float* trap, const float* q_bias, const float* k_bias,
                                  const float* cos, const float* sin, const float* d_skip,
                                  const float* z, int backend, int threading, float* out,
                                  void* stream) {
  if (dims && dims->rank != 1)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "the non-causal sum is SISO (rank %zu given)",
                dims->rank);
  // forward writes out; backward adds its strictly-later terms
  if (int rc = mamba3_call(dims, q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z,
                           nullptr, nullptr, nullptr, 0, backend, threading, out, nullptr,
                           nullptr, stream, true))
    return rc;
  return mamba3_call(dims, q, k, v, adt, dt, trap, q_bias, k_bias, cos, sin, d_skip, z,
                     nullptr, nullptr, nullptr, 1, backend, threading, out, nullptr, nullptr,
                     stream, true, nullptr, 0, true);
}

int arm_scan_mamba3_angles_f32(const float* angles, const float* dt, size_t batch, size_t len,
                               size_t heads, size_t n_angles, size_t half, float* cos,
                               float* sin, void* stream) {
  if (!angles || !dt || !cos || !sin)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (!batch || !len || !heads || !half)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "a dimension is zero");
  if (n_angles > half)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "n_angles (%zu) exceeds the pairs (%zu)", n_angles,
                half);
  if (!prod_ok({batch, len, heads, half}) || len > (1u << 30) || heads > (1u << 30))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "dims overflow");
  return run(armscan::m3_angles_to_cos_sin(angles, dt, batch, len, heads, n_angles, half, cos,
                                           sin, (hipStream_t)stream),
             "angle pre-pass launch");
}

int arm_scan_ss2d_f32(const ArmSS2DDims* dims, const float* u, const float* delta,
                      const float* a, const float* b4, const float* c4, const float* d_skip,
                      const float* z, const float* delta_bias, int delta_softplus, int merge,
                      float* out, float* last_states, void* stream) {
  if (!dims || !u || !delta || !a || !b4 || !c4 || !out)
    return fail(ARM_SCAN_ERR_NULL_POINTER, "a required pointer is null");
  if (merge < 0 || merge > 2) return fail(ARM_SCAN_ERR_BAD_ENUM, "bad merge enum %d", merge);
  const ArmSS2DDims& d = *dims;
  if (!d.batch || !d.dim || !d.height || !d.width || !d.state)
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "a dimension is zero");
  if (!prod_ok({4, d.batch, d.dim, d.height, d.width}) ||
      !prod_ok({4, d.batch, d.state, d.height, d.width}) || d.height > (1u << 20) ||
      d.width > (1u << 20) || d.batch * d.dim > (1u << 30))
    return fail(ARM_SCAN_ERR_INVALID_DIMS, "dims overflow or too large");
  hipStream_t st = (hipStream_t)stream;
  const size_t H = d.height, W = d.width, L = H * W;
  const size_t plane = d.batch * d.dim * L;    // one (b, d, H, W) plane
  const size_t bcp = d.batch * d.state * L;    // one direction's B or C
  const size_t bdn = d.batch * d.dim * d.state;

  armscan::M1Problem p{};
  p.batch = d.batch; p.dim = d.dim; p.len = L; p.state = d.state; p.groups = 1;
  p.A = a; p.D = d_skip; p.bias = delta_bias; p.softplus = delta_softplus != 0;

  float* ls0 = last_states;
  auto last_of = [&](int k) { return ls0 ? ls0 + (size_t)k * bdn : nullptr; };
  {
    armscan::M1Problem q = p;
    q.u = u; q.delta = delta; q.z = z;
    q.B = b4; q.C = c4; q.out = out;
    if (armscan::m1_jobs_supported(q)) {
      // One launch for the four directions. The column directions scan column-major
      // copies of u, delta, z and of their B/C (one batched transpose) and write
      // their planes column-major; the merge (or, with merge none, a second batched
      // transpose) brings them back onto the grid.
      const bool none = merge == 0;
      const size_t n_scratch = (z ? 3 : 2) * plane + 4 * bcp + 2 * plane + (none ? 0 : plane);
      float* scratch = nullptr;
      hipError_t e = armscan::stream_alloc((void**)&scratch, n_scratch * sizeof(float), st);
      if (e != hipSuccess) return hip_fail(e, "ss2d scratch allocation");
      float* uT = scratch;
      float* dT = uT + plane;
      float* zT = z ? dT + plane : nullptr;
      float* bT = (z ? zT : dT) + plane;  // b4[2], b4[3], c4[2], c4[3] column-major
      float* q2 = bT + 4 * bcp;           // column-forward plane (column-major)
      float* q3 = q2 + plane;             // column-backward plane
      float* p1 = none ? out + plane : q3 + plane;
      const long long bd = (long long)(d.batch * d.dim), bn = (long long)(d.batch * d.state);
      armscan::TransposeSpec tin[7] = {{u, uT, bd},
                                       {delta, dT, bd},
                                       {b4 + 2 * bcp, bT, bn},
                                       {b4 + 3 * bcp, bT + bcp, bn},
                                       {c4 + 2 * bcp, bT + 2 * bcp, bn},
                                       {c4 + 3 * bcp, bT + 3 * bcp, bn},
                                       {z, zT, bd}};
      e = armscan::transpose_batch(tin, z ? 7 : 6, (int)H, (int)W, st);
      if (e == hipSuccess) {
        const armscan::M1JobSpec jobs[4] = {
            {u, delta, z, b4, c4, out, last_of(0), 0},
            {u, delta, z, b4 + bcp, c4 + bcp, p1, last_of(1), 1},
            {uT, dT, zT, bT, bT + 2 * bcp, q2, last_of(2), 0},
            {uT, dT, zT, bT + bcp, bT + 3 * bcp, q3, last_of(3), 1}};
        e = armscan::m1_scan_jobs(q, jobs, 4, st);
      }
      if (e == hipSuccess) {
        if (none) {
          const armscan::TransposeSpec tout[2] = {{q2, out + 2 * plane, bd},
                                                  {q3, out + 3 * plane, bd}};
          e = armscan::transpose_batch(tout, 2, (int)W, (int)H, st);
        } else {
          e = armscan::merge4_transposed(out, p1, q2, q3, bd, (int)H, (int)W,
                                         merge == 2 ? 0.25f : 1.0f, st);
        }
      }
      int rc = e == hipSuccess ? ARM_SCAN_OK : hip_fail(e, "ss2d launch");
      const hipError_t fe = hipFreeAsync(scratch, st);
      if (rc == ARM_SCAN_OK && fe != hipSuccess) rc = hip_fail(fe, "ss2d scratch free");
      return rc;
    }
  }

  // Otherwise: the column-major views of u, delta, z and the column directions'
  // B/C, plus the column pair's outputs before they are transposed back.
  const size_t n_scratch = plane * (z ? 3 : 2) + 4 * bcp + 2 * plane;
  float* scratch = nullptr;
  hipError_t e = armscan::stream_alloc((void**)&scratch, n_scratch * sizeof(float), st);
  if (e != hipSuccess) return hip_fail(e, "ss2d scratch allocation");
  float* uT = scratch;
  float* dT = uT + plane;
  float* zT = z ? dT + plane : nullptr;
  float* bT = (z ? zT : dT) + plane;  // b4[2], b4[3], c4[2], c4[3] transposed
  float* colf = bT + 4 * bcp;
  float* colb = colf + plane;

  // One traversal pair (forward + reverse over the same ordering). `sum` asks
  // for of = fwd + bwd (ob unused); otherwise of / ob receive the two planes.
  auto pair = [&](const float* uu, const float* dd, const float* zz, const float* Bf,
                  const float* Bb, const float* Cf, const float* Cb, float* of, float* ob,
                  float* lf, float* lb, bool sum, float* tmp) -> hipError_t {
    armscan::M1Problem q = p;
    q.u = uu; q.delta = dd; q.z = zz;
    q.B = Bf; q.C = Cf; q.B2 = Bb; q.C2 = Cb;
    if (armscan::m1_bidir_fusable(q)) {
      q.out = of; q.out2 = sum ? nullptr : ob; q.last = lf; q.last2 = lb;
      q.merge = sum ? 1 : 0;
      return armscan::m1_bidir(q, st);
    }
    q.B2 = q.C2 = nullptr;
    q.out = of; q.last = lf; q.reverse = 0;
    hipError_t r = armscan::m1_scan(q, st);
    if (r != hipSuccess) return r;
    q.B = Bb; q.C = Cb; q.out = sum ? tmp : ob; q.last = lb; q.reverse = 1;
    r = armscan::m1_scan(q, st);
    if (r != hipSuccess || !sum) return r;
    return armscan::add_inplace(of, tmp, (long long)plane, st);
  };

  float* ls = last_states;
  auto last_at = [&](int k) { return ls ? ls + (size_t)k * bdn : nullptr; };
  const bool none = merge == 0;
  int rc = ARM_SCAN_OK;
  do {
    // column-major views for the column directions
    const long long bd = (long long)(d.batch * d.dim), bn = (long long)(d.batch * d.state);
    if ((e = armscan::transpose_hw(u, uT, bd, (int)H, (int)W, false, st))) break;
    if ((e = armscan::transpose_hw(delta, dT, bd, (int)H, (int)W, false, st))) break;
    if (z && (e = armscan::transpose_hw(z, zT, bd, (int)H, (int)W, false, st))) break;
    for (int kk = 0; kk < 2 && !e; ++kk) {
      e = armscan::transpose_hw(b4 + (2 + kk) * bcp, bT + kk * bcp, bn, (int)H, (int)W, false,
                                st);
      if (!e)
        e = armscan::transpose_hw(c4 + (2 + kk) * bcp, bT + (2 + kk) * bcp, bn, (int)H, (int)W,
                                  false, st);
    }
    if (e) break;
    // row pair over the row-major flattening: planes 0 / 1, or their sum into out
    e = pair(u, delta, z, b4, b4 + bcp, c4, c4 + bcp, out, none ? out + plane : nullptr,
             last_at(0), last_at(1), !none, colf);
    if (e) break;
    // column pair on the transposed grid, then back to (H, W)
    e = pair(uT, dT, zT, bT, bT + bcp, bT + 2 * bcp, bT + 3 * bcp, colf, none ? colb : nullptr,
             last_at(2), last_at(3), !none, colb);
    if (e) break;
    if (none) {
      if ((e = armscan::transpose_hw(colf, out + 2 * plane, bd, (int)W, (int)H, false, st)))
        break;
      e = armscan::transpose_hw(colb, out + 3 * plane, bd, (int)W, (int)H, false, st);
    } else {
      if ((e = armscan::transpose_hw(colf, out, bd, (int)W, (int)H, true, st))) break;
      if (merge == 2) e = armscan::scale_inplace(out, (long long)plane, 0.25f, st);
    }
  } while (false);
  if (e != hipSuccess) rc = hip_fail(e, "ss2d launch");
  hipError_t fe = hipFreeAsync(scratch, st);
  if (rc == ARM_SCAN_OK && fe != hipSuccess) rc = hip_fail(fe, "ss2d scratch free");
  return rc;
}

}  // extern "C"
