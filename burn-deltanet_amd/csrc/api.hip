// The C ABI (include/deltanet_core.h): argument checks that mirror the
// reference's assertions, workspace management and kernel dispatch.

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstring>
#include <initializer_list>
#include <mutex>
#include <string>
#include <vector>

#include "dn_common.hpp"

namespace dn {
namespace {

thread_local std::string g_last_error;

int fail(int code, const std::string& msg) {
  g_last_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(DN_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

// Library-managed workspace: grow-only, one buffer per device, freed at exit.
struct Pool {
  std::mutex mu;
  std::vector<void*> ptr;
  std::vector<size_t> size;
  ~Pool() {
    for (void* p : ptr)
      if (p) (void)hipFree(p);
  }
};
Pool g_pool;

// The pool is one buffer per device: calls that use it on two streams at once
// share it (they race), and growing it frees the old buffer after a device
// synchronisation, which a stream under HIP graph capture must not see (a
// captured graph would keep the freed pointer). Growth is therefore refused
// during capture (hipErrorStreamCaptureUnsupported); callers that capture or
// run several streams pass their own workspace.
hipError_t pool_get(size_t bytes, void** out, hipStream_t stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(g_pool.mu);
  if (size_t(dev) >= g_pool.ptr.size()) {
    g_pool.ptr.resize(size_t(dev) + 1, nullptr);
    g_pool.size.resize(size_t(dev) + 1, 0);
  }
  if (g_pool.size[size_t(dev)] < bytes) {
    hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
    if ((e = hipStreamIsCapturing(stream, &cap)) != hipSuccess) return e;
    if (cap != hipStreamCaptureStatusNone) return hipErrorStreamCaptureUnsupported;
    // Callers on this device may still be using the old buffer on their
    // streams; drain the device before it is replaced.
    if (g_pool.ptr[size_t(dev)]) {
      if ((e = hipDeviceSynchronize()) != hipSuccess) return e;
      (void)hipFree(g_pool.ptr[size_t(dev)]);
      g_pool.ptr[size_t(dev)] = nullptr;
      g_pool.size[size_t(dev)] = 0;
    }
    void* p = nullptr;
    if ((e = hipMalloc(&p, bytes)) != hipSuccess) return e;
    g_pool.ptr[size_t(dev)] = p;
    g_pool.size[size_t(dev)] = bytes;
  }
  *out = g_pool.ptr[size_t(dev)];
  return hipSuccess;
}

// Scratch of dn_chunk_fwd_noalloc: a file-scope device array, so that entry
// point allocates nothing. Each device that loads the library holds its own
// copy (DN_NOALLOC_SCRATCH_BYTES) until the process ends. In host code
// `scratch` only stands in for the symbol; its device address, per device,
// comes from hipGetSymbolAddress (scratch_ptr) and is what kernels receive.
__device__ __align__(256) unsigned char scratch[DN_NOALLOC_SCRATCH_BYTES];

// The calling thread's current device's address of `scratch`, looked up once
// per device (with that device current) and kept.
hipError_t scratch_ptr(void** out) {
  static std::mutex mu;
  static std::vector<void*> ptrs;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  if (size_t(dev) >= ptrs.size()) ptrs.resize(size_t(dev) + 1, nullptr);
  if (!ptrs[size_t(dev)]) {
    void* p = nullptr;
    if ((e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch))) != hipSuccess) return e;
    ptrs[size_t(dev)] = p;
  }
  *out = ptrs[size_t(dev)];
  return hipSuccess;
}

bool valid_dtype(int t) { return t == DN_F32 || t == DN_BF16; }

// The product of the extents, or -1 when one of them exceeds INT32_MAX (the
// kernels' index width) or the product overflows.
int64_t extent(std::initializer_list<int64_t> xs) {
  int64_t n = 1;
  for (const int64_t x : xs)
    if (x > INT32_MAX || __builtin_mul_overflow(n, x, &n)) return -1;
  return n;
}
// An extent that is unrepresentable or reaches `limit`.
bool too_large(std::initializer_list<int64_t> xs, int64_t limit) {
  const int64_t n = extent(xs);
  return n < 0 || n >= limit;
}

// The reference's shape/gate checks (path.rs:177-208, recurrent.rs:51-54).
int check_common(int64_t batch, int64_t sequence, int64_t nheads, int64_t K, int64_t V,
                 int64_t ew, int64_t ww, int64_t dw, int32_t has_gate) {
  if (sequence < 1) return fail(DN_ERR_SEQUENCE, "sequence length must be at least 1");
  if (batch < 1 || nheads < 1 || K < 1 || V < 1)
    return fail(DN_ERR_SHAPE, "batch, nheads, head_k_dim and head_v_dim must be at least 1");
  // Every extent fits the kernels' 32-bit index arithmetic, and the largest
  // tensor stays below 2^40 elements (checked factor by factor, so the
  // product cannot overflow on the way).
  if (too_large({batch, sequence, nheads, K > V ? K : V}, int64_t(1) << 40))
    return fail(DN_ERR_SHAPE, "tensor too large");
  if (!(ew == 1 || ew == K))
    return fail(DN_ERR_GATE_WIDTH, "erase gate: last axis must be 1 or " + std::to_string(K) +
                                       ", got " + std::to_string(ew));
  if (!(ww == 1 || ww == V))
    return fail(DN_ERR_GATE_WIDTH, "write gate: last axis must be 1 or " + std::to_string(V) +
                                       ", got " + std::to_string(ww));
  if (has_gate && !(dw == 1 || dw == K))
    return fail(DN_ERR_GATE_WIDTH, "forget gate: last axis must be 1 or " + std::to_string(K) +
                                       ", got " + std::to_string(dw));
  return DN_OK;
}

float resolve_scale(double scale, int64_t K) {
  return std::isnan(scale) ? float(1.0 / std::sqrt(double(K))) : float(scale);
}

Dims make_dims(int64_t B, int64_t S, int64_t H, int64_t K, int64_t V, int64_t ew, int64_t ww,
               int64_t dw, int32_t has_gate, int32_t L, double scale) {
  Dims d;
  d.B = int(B);
  d.S = int(S);
  d.H = int(H);
  d.K = int(K);
  d.V = int(V);
  d.ew = int(ew);
  d.ww = int(ww);
  d.dw = has_gate ? int(dw) : 0;
  d.L = L;
  d.N = int((S + L - 1) / L);
  d.scale = resolve_scale(scale, K);
  return d;
}

// NaN/Inf guard over a list of (pointer, count, dtype); synchronises.
struct Guarded {
  const void* p;
  size_t n;
  int dtype;
};

// One device int per device for the guard flag, allocated on first use.
hipError_t guard_flag(int** out) {
  static std::mutex mu;
  static std::vector<int*> flags;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  if (size_t(dev) >= flags.size()) flags.resize(size_t(dev) + 1, nullptr);
  if (!flags[size_t(dev)]) {
    void* p = nullptr;
    if ((e = hipMalloc(&p, sizeof(int))) != hipSuccess) return e;
    flags[size_t(dev)] = static_cast<int*>(p);
  }
  *out = flags[size_t(dev)];
  return hipSuccess;
}

// The give-up counter of the bounded cross-workgroup waits (the fused output
// norm's exchange), one device int per device, zeroed when allocated.
hipError_t give_up_counter(int** out) {
  static std::mutex mu;
  static std::vector<int*> counters;
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  std::lock_guard<std::mutex> lock(mu);
  if (size_t(dev) >= counters.size()) counters.resize(size_t(dev) + 1, nullptr);
  if (!counters[size_t(dev)]) {
    void* p = nullptr;
    if ((e = hipMalloc(&p, sizeof(int))) != hipSuccess) return e;
    if ((e = hipMemset(p, 0, sizeof(int))) != hipSuccess) return e;
    counters[size_t(dev)] = static_cast<int*>(p);
  }
  *out = counters[size_t(dev)];
  return hipSuccess;
}

// Polls before an exchange wait gives up: about 0.2 s of 128-cycle sleeps,
// far beyond the microseconds a resident partner takes.
constexpr int kNormSpin = 1 << 22;

int nonfinite_check(const std::vector<Guarded>& list, hipStream_t stream, const char* when) {
  int* flag = nullptr;
  hipError_t e = guard_flag(&flag);
  if (e != hipSuccess) return hip_fail(e, "guard flag allocation");
  int host = 0;
  if ((e = hipMemcpyAsync(flag, &host, sizeof(int), hipMemcpyHostToDevice, stream)) !=
      hipSuccess)
    return hip_fail(e, "guard flag upload");
  for (const Guarded& g : list)
    if (g.p && g.n)
      if ((e = launch_nonfinite_scan(g.p, g.n, g.dtype, flag, stream)) != hipSuccess)
        return hip_fail(e, "nonfinite scan launch");
  if ((e = hipMemcpyAsync(&host, flag, sizeof(int), hipMemcpyDeviceToHost, stream)) !=
      hipSuccess)
    return hip_fail(e, "guard flag readback");
  if ((e = hipStreamSynchronize(stream)) != hipSuccess) return hip_fail(e, "guard sync");
  if (host) return fail(DN_ERR_NONFINITE, std::string("NaN or Inf found in the ") + when);
  return DN_OK;
}

// The generic kernels index a chunk's L×L and L×head-dim tiles with 32-bit
// integers (a chunk longer than the sequence is padded to its full length).
int check_chunk_len(int64_t L, int64_t K, int64_t V) {
  if (L < 1) return fail(DN_ERR_CHUNK_LEN, "chunk_len must be at least 1");
  if (L * L > INT32_MAX || L * (K > V ? K : V) > INT32_MAX)
    return fail(DN_ERR_CHUNK_LEN, "chunk_len too large: chunk_len² and chunk_len·head dim must "
                                  "stay below 2^31");
  return DN_OK;
}

int check_fwd(const dn_chunk_fwd_args* a) {
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  if (int rc = check_common(a->batch, a->sequence, a->nheads, a->head_k_dim, a->head_v_dim,
                            a->erase_width, a->write_width, a->decay_width, a->has_gate))
    return rc;
  if (int rc = check_chunk_len(a->chunk_len, a->head_k_dim, a->head_v_dim)) return rc;
  if (!valid_dtype(a->qkv_dtype) || !valid_dtype(a->y_dtype))
    return fail(DN_ERR_DTYPE, "dtype must be DN_F32 or DN_BF16");
  if (!a->q || !a->k || !a->v || !a->erase || !a->write || !a->state_in || !a->y ||
      !a->state_out || (a->has_gate && !a->g))
    return fail(DN_ERR_NULL, "a required tensor pointer is NULL");
  return DN_OK;
}

int check_bwd(const dn_chunk_bwd_args* a) {
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  if (int rc = check_common(a->batch, a->sequence, a->nheads, a->head_k_dim, a->head_v_dim,
                            a->erase_width, a->write_width, a->decay_width, a->has_gate))
    return rc;
  if (int rc = check_chunk_len(a->chunk_len, a->head_k_dim, a->head_v_dim)) return rc;
  if (!valid_dtype(a->qkv_dtype) || !valid_dtype(a->grad_dtype))
    return fail(DN_ERR_DTYPE, "dtype must be DN_F32 or DN_BF16");
  if (!a->d_y || !a->q || !a->k || !a->v || !a->erase || !a->write || !a->state_in ||
      !a->d_q || !a->d_k || !a->d_v || !a->d_erase || !a->d_write || !a->d_state ||
      (a->has_gate && (!a->g || !a->d_g)))
    return fail(DN_ERR_NULL, "a required tensor pointer is NULL");
  return DN_OK;
}

bool mfma_requested(int algo) { return algo == DN_ALGO_MFMA || algo == DN_ALGO_MFMA_FUSED; }

// The MFMA kernels walk 64-token chunks. Without a per-key-channel forget
// gate the chunk length orders the roundings and nothing else: the chunk
// form and the token recurrence are one function (path.rs:15-19, 46-49), so
// a request for another chunk length runs those kernels at 64. With a
// per-channel forget gate the reference's block decay clamps exponents
// inside a chunk (decay.rs:39-60), which makes its values in that regime
// depend on where chunks start: such requests keep their own chunk length
// (and, at lengths other than 64, the generic kernels).
constexpr int kMfmaChunk = 64;
Dims mfma_dims(const Dims& d) {
  if (d.L == kMfmaChunk || (d.dw == d.K && d.K > 1)) return d;
  Dims m = d;
  m.L = kMfmaChunk;
  m.N = (d.S + kMfmaChunk - 1) / kMfmaChunk;
  return m;
}
// The dims a call runs with: its own for the generic kernels.
Dims run_dims(const Dims& d, int algo) { return algo == DN_ALGO_GENERIC ? d : mfma_dims(d); }

// The MFMA kernels read q and k in 16-byte words and v in 4-byte words; a
// tensor view that starts off those boundaries takes the generic kernels.
bool mfma_aligned(const void* q, const void* k, const void* v) {
  return reinterpret_cast<uintptr_t>(q) % 16 == 0 && reinterpret_cast<uintptr_t>(k) % 16 == 0 &&
         reinterpret_cast<uintptr_t>(v) % 4 == 0;
}

// The forward's kernels: DN_ALGO_GENERIC, DN_ALGO_MFMA (intra + scan) or,
// on request only, DN_ALGO_MFMA_FUSED (one kernel; at BASELINE config 2 on
// a warm MI355X 0.47 ms against the two kernels' 0.38-0.39 ms).
int fwd_algo(const dn_chunk_fwd_args* a, const Dims& d0) {
  if (a->algo == DN_ALGO_GENERIC) return DN_ALGO_GENERIC;
  const Dims d = mfma_dims(d0);
  const bool fits =
      mfma_fwd_supported(d, a->qkv_dtype, a->y_dtype) && mfma_aligned(a->q, a->k, a->v);
  if (a->algo == DN_ALGO_MFMA_FUSED)
    return fits && fused_fwd_supported(d, a->qkv_dtype) ? DN_ALGO_MFMA_FUSED
                                                         : DN_ERR_UNSUPPORTED;
  if (a->algo == DN_ALGO_MFMA) return fits ? DN_ALGO_MFMA : DN_ERR_UNSUPPORTED;
  return fits ? DN_ALGO_MFMA : DN_ALGO_GENERIC;
}

size_t fwd_workspace(const Dims& d, int algo) {
  if (algo == DN_ALGO_GENERIC) return generic_fwd_workspace(d);
  return mfma_fwd_workspace(d, algo == DN_ALGO_MFMA_FUSED);
}

Dims bwd_dims(const dn_chunk_bwd_args* a) {
  return make_dims(a->batch, a->sequence, a->nheads, a->head_k_dim, a->head_v_dim,
                   a->erase_width, a->write_width, a->decay_width, a->has_gate, a->chunk_len,
                   a->scale);
}

// MFMA: the two scans of the backward on bf16 MFMA (the forward MFMA path's
// shapes, bf16 q/k/v), and for head_v_dim 64 or 128 the chunk-local
// gradients too; otherwise those stay on the generic fp32 kernel.
// The backward's MFMA kernels also read d_y in 16-byte words.
int bwd_algo(const dn_chunk_bwd_args* a, const Dims& d0) {
  if (a->algo == DN_ALGO_GENERIC) return DN_ALGO_GENERIC;
  const Dims d = mfma_dims(d0);
  const bool fits = mfma_bwd_supported(d, a->qkv_dtype) && mfma_aligned(a->q, a->k, a->v) &&
                    reinterpret_cast<uintptr_t>(a->d_y) % 16 == 0;
  if (mfma_requested(a->algo)) return fits ? DN_ALGO_MFMA : DN_ERR_UNSUPPORTED;
  return fits ? DN_ALGO_MFMA : DN_ALGO_GENERIC;
}

bool bwd_all_mfma(const Dims& d, int qkv_dtype, int algo) {
  return algo == DN_ALGO_MFMA && mfma_chunk_bwd_supported(d, qkv_dtype);
}

// Per-chunk states and state cotangents, fp32 [G][K][V] each.
size_t bwd_state_bytes(const Dims& d) {
  return align_up(size_t(d.B) * d.N * d.H * d.K * d.V * sizeof(float), 256);
}

size_t bwd_workspace(const Dims& d, int algo, int qkv_dtype) {
  if (bwd_all_mfma(d, qkv_dtype, algo))
    return 2 * bwd_state_bytes(d) + align_up(mfma_bwd_workspace(d), 256) +
           mfma_chunk_bwd_partials(d);
  return align_up(generic_bwd_workspace(d), 256) + (algo == DN_ALGO_MFMA ? mfma_bwd_workspace(d) : 0);
}

}  // namespace
}  // namespace dn

using namespace dn;

extern "C" {

const char* dn_last_error(void) { return g_last_error.c_str(); }

const char* dn_version(void) { return "deltanet-mi355x 0.1.0 (gfx950)"; }

int dn_chunk_fwd_algo(const dn_chunk_fwd_args* a) {
  if (int rc = check_fwd(a)) return rc;
  Dims d = make_dims(a->batch, a->sequence, a->nheads, a->head_k_dim, a->head_v_dim,
                     a->erase_width, a->write_width, a->decay_width, a->has_gate, a->chunk_len,
                     a->scale);
  return fwd_algo(a, d);
}

size_t dn_chunk_fwd_workspace_bytes(const dn_chunk_fwd_args* a) {
  if (check_fwd(a)) return 0;
  Dims d = make_dims(a->batch, a->sequence, a->nheads, a->head_k_dim, a->head_v_dim,
                     a->erase_width, a->write_width, a->decay_width, a->has_gate, a->chunk_len,
                     a->scale);
  const int algo = fwd_algo(a, d);
  return algo < 0 ? 0 : fwd_workspace(run_dims(d, algo), algo);
}

int dn_chunk_fwd(const dn_chunk_fwd_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (int rc = check_fwd(a)) return rc;
  Dims d = make_dims(a->batch, a->sequence, a->nheads, a->head_k_dim, a->head_v_dim,
                     a->erase_width, a->write_width, a->decay_width, a->has_gate, a->chunk_len,
                     a->scale);
  const int algo = fwd_algo(a, d);
  if (algo < 0)
    return fail(DN_ERR_UNSUPPORTED, "the requested MFMA path does not cover this shape/dtype");
  d = run_dims(d, algo);
  const size_t need = fwd_workspace(d, algo);
  void* ws = a->workspace;
  if (ws) {
    if (a->workspace_bytes < need)
      return fail(DN_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) +
                                        " bytes");
  } else if (need) {
    hipError_t e = pool_get(need, &ws, stream);
    if (e != hipSuccess) return hip_fail(e, "workspace allocation");
  }
  const size_t nq = size_t(d.B) * d.S * d.H, ns = size_t(d.B) * d.H * d.K * d.V;
  if (a->check_finite) {
    std::vector<Guarded> in = {{a->q, nq * d.K, a->qkv_dtype},
                               {a->k, nq * d.K, a->qkv_dtype},
                               {a->v, nq * d.V, a->qkv_dtype},
                               {a->erase, nq * d.ew, DN_F32},
                               {a->write, nq * d.ww, DN_F32},
                               {a->has_gate ? a->g : nullptr, nq * d.dw, DN_F32},
                               {a->state_in, ns, DN_F32}};
    if (int rc = nonfinite_check(in, stream, "inputs")) return rc;
  }
  hipError_t e;
  if (algo != DN_ALGO_GENERIC)
    e = mfma_fwd(d, a->y_dtype, a->q, a->k, a->v, a->erase, a->write,
                 a->has_gate ? a->g : nullptr, a->state_in, a->y, a->state_out, ws, stream,
                 algo == DN_ALGO_MFMA_FUSED);
  else
    e = generic_fwd(d, a->qkv_dtype, a->y_dtype, a->q, a->k, a->v, a->erase, a->write,
                    a->has_gate ? a->g : nullptr, a->state_in, a->y, a->state_out, ws, stream);
  if (e != hipSuccess) return hip_fail(e, "dn_chunk_fwd launch");
  if (a->check_finite) {
    std::vector<Guarded> out = {{a->y, nq * d.V, a->y_dtype}, {a->state_out, ns, DN_F32}};
    if (int rc = nonfinite_check(out, stream, "outputs")) return rc;
  }
  return DN_OK;
}

int dn_chunk_fwd_noalloc(const dn_chunk_fwd_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (int rc = check_fwd(a)) return rc;
  if (a->check_finite)
    return fail(DN_ERR_UNSUPPORTED,
                "dn_chunk_fwd_noalloc does not run the NaN/Inf guard (its flag is allocated and "
                "read back); use dn_chunk_fwd for check_finite");
  Dims d = make_dims(a->batch, a->sequence, a->nheads, a->head_k_dim, a->head_v_dim,
                     a->erase_width, a->write_width, a->decay_width, a->has_gate, a->chunk_len,
                     a->scale);
  const int algo = fwd_algo(a, d);
  if (algo < 0)
    return fail(DN_ERR_UNSUPPORTED, "the requested MFMA path does not cover this shape/dtype");
  d = run_dims(d, algo);
  const size_t need = fwd_workspace(d, algo);
  if (need > size_t(DN_NOALLOC_SCRATCH_BYTES))
    return fail(DN_ERR_WORKSPACE,
                "dn_chunk_fwd_noalloc: these arguments need " + std::to_string(need) +
                    " bytes of scratch, above its maximum of " +
                    std::to_string(size_t(DN_NOALLOC_SCRATCH_BYTES)) +
                    "; call dn_chunk_fwd with a workspace instead");
  void* ws = nullptr;
  hipError_t e = scratch_ptr(&ws);
  if (e != hipSuccess) return hip_fail(e, "scratch address");
  // Every byte of scratch a forward kernel reads was written earlier in the
  // same call (no counters or partial sums), so nothing is cleared first.
  if (algo != DN_ALGO_GENERIC)
    e = mfma_fwd(d, a->y_dtype, a->q, a->k, a->v, a->erase, a->write,
                 a->has_gate ? a->g : nullptr, a->state_in, a->y, a->state_out, ws, stream,
                 algo == DN_ALGO_MFMA_FUSED);
  else
    e = generic_fwd(d, a->qkv_dtype, a->y_dtype, a->q, a->k, a->v, a->erase, a->write,
                    a->has_gate ? a->g : nullptr, a->state_in, a->y, a->state_out, ws, stream);
  if (e != hipSuccess) return hip_fail(e, "dn_chunk_fwd_noalloc launch");
  return DN_OK;
}

namespace {

int check_fwd_norm(const dn_chunk_fwd_out_norm_args* a) {
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  if (int rc = check_fwd(&a->fwd)) return rc;
  if (!a->weight) return fail(DN_ERR_NULL, "norm weight is NULL");
  if (!(a->eps >= 0.0) || !std::isfinite(a->eps))
    return fail(DN_ERR_SHAPE, "eps must be finite and non-negative");
  if (a->fwd.head_v_dim > DN_OUT_NORM_MAX_HEAD_DIM)
    return fail(DN_ERR_UNSUPPORTED,
                "the output norm supports head_v_dim up to " +
                    std::to_string(DN_OUT_NORM_MAX_HEAD_DIM));
  if (a->gate) {
    if (!valid_dtype(a->gate_dtype)) return fail(DN_ERR_DTYPE, "dtype must be DN_F32 or DN_BF16");
    if (a->gate_stride < a->fwd.nheads * a->fwd.head_v_dim)
      return fail(DN_ERR_SHAPE, "gate_stride must cover nheads * head_v_dim");
  }
  return DN_OK;
}

// The fused norm reads the gate, in y's dtype, and y in words of 4 values
// at 32-bit offsets within a chunk's 64 token rows.
bool norm_fusable(const dn_chunk_fwd_out_norm_args* a) {
  const size_t word = a->fwd.y_dtype == DN_BF16 ? 8 : 16;
  const bool gate_ok = !a->gate || (a->gate_dtype == a->fwd.y_dtype &&
                                    reinterpret_cast<uintptr_t>(a->gate) % word == 0 &&
                                    a->gate_stride % 4 == 0 && a->gate_stride < (int64_t(1) << 25));
  // The norm-applying scans cover head_k_dim 64 and 128.
  return gate_ok && reinterpret_cast<uintptr_t>(a->fwd.y) % word == 0 && a->fwd.head_k_dim <= 128;
}

}  // namespace

size_t dn_chunk_fwd_out_norm_workspace_bytes(const dn_chunk_fwd_out_norm_args* a) {
  if (check_fwd_norm(a)) return 0;
  const dn_chunk_fwd_args* f = &a->fwd;
  Dims d = make_dims(f->batch, f->sequence, f->nheads, f->head_k_dim, f->head_v_dim,
                     f->erase_width, f->write_width, f->decay_width, f->has_gate, f->chunk_len,
                     f->scale);
  const int algo = fwd_algo(f, d);
  if (algo < 0) return 0;
  d = run_dims(d, algo);
  return a->in_scan && algo == DN_ALGO_MFMA && norm_fusable(a) ? mfma_fwd_norm_workspace(d)
                                                               : fwd_workspace(d, algo);
}

int dn_chunk_fwd_out_norm(const dn_chunk_fwd_out_norm_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (int rc = check_fwd_norm(a)) return rc;
  const dn_chunk_fwd_args* f = &a->fwd;
  Dims d = make_dims(f->batch, f->sequence, f->nheads, f->head_k_dim, f->head_v_dim,
                     f->erase_width, f->write_width, f->decay_width, f->has_gate, f->chunk_len,
                     f->scale);
  const int algo = fwd_algo(f, d);
  if (algo < 0)
    return fail(DN_ERR_UNSUPPORTED, "the requested MFMA path does not cover this shape/dtype");
  d = run_dims(d, algo);
  const bool in_scan = a->in_scan && algo == DN_ALGO_MFMA && norm_fusable(a);
  const size_t need = in_scan ? mfma_fwd_norm_workspace(d) : fwd_workspace(d, algo);
  void* ws = f->workspace;
  if (ws) {
    if (f->workspace_bytes < need)
      return fail(DN_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) +
                                        " bytes");
  } else if (need) {
    hipError_t e = pool_get(need, &ws, stream);
    if (e != hipSuccess) return hip_fail(e, "workspace allocation");
  }
  const size_t nq = size_t(d.B) * d.S * d.H, ns = size_t(d.B) * d.H * d.K * d.V;
  if (f->check_finite) {
    std::vector<Guarded> in = {{f->q, nq * d.K, f->qkv_dtype},
                               {f->k, nq * d.K, f->qkv_dtype},
                               {f->v, nq * d.V, f->qkv_dtype},
                               {f->erase, nq * d.ew, DN_F32},
                               {f->write, nq * d.ww, DN_F32},
                               {f->has_gate ? f->g : nullptr, nq * d.dw, DN_F32},
                               {f->state_in, ns, DN_F32},
                               {a->weight, size_t(d.V), DN_F32}};
    if (int rc = nonfinite_check(in, stream, "inputs")) return rc;
  }
  const float* g = f->has_gate ? f->g : nullptr;
  hipError_t e = hipErrorCooperativeLaunchTooLarge;
  if (in_scan) {
    int* fault = nullptr;
    if ((e = give_up_counter(&fault)) != hipSuccess) return hip_fail(e, "wait counter");
    FwdNorm nm{a->gate, (long long)a->gate_stride, a->weight, float(a->eps), fault, kNormSpin};
    e = mfma_fwd_norm(d, f->y_dtype, f->q, f->k, f->v, f->erase, f->write, g, f->state_in, f->y,
                      f->state_out, ws, nm, stream);
  }
  if (e == hipErrorCooperativeLaunchTooLarge) {
    // The forward, then the norm in place on y.
    if (algo != DN_ALGO_GENERIC)
      e = mfma_fwd(d, f->y_dtype, f->q, f->k, f->v, f->erase, f->write, g, f->state_in, f->y,
                   f->state_out, ws, stream, algo == DN_ALGO_MFMA_FUSED);
    else
      e = generic_fwd(d, f->qkv_dtype, f->y_dtype, f->q, f->k, f->v, f->erase, f->write, g,
                      f->state_in, f->y, f->state_out, ws, stream);
    if (e == hipSuccess) {
      dn_out_norm_args n{};
      n.tokens = int64_t(d.B) * d.S;
      n.nheads = d.H;
      n.head_v_dim = d.V;
      n.gate_stride = a->gate_stride;
      n.eps = a->eps;
      n.x_dtype = n.out_dtype = f->y_dtype;
      n.gate_dtype = a->gate_dtype;
      n.x = f->y;
      n.gate = a->gate;
      n.weight = a->weight;
      n.out = f->y;
      e = launch_out_norm(n, stream);
    }
  }
  if (e != hipSuccess) return hip_fail(e, "dn_chunk_fwd_out_norm launch");
  if (f->check_finite) {
    std::vector<Guarded> out = {{f->y, nq * d.V, f->y_dtype}, {f->state_out, ns, DN_F32}};
    if (int rc = nonfinite_check(out, stream, "outputs")) return rc;
  }
  return DN_OK;
}

int64_t dn_wait_give_ups(void) {
  g_last_error.clear();
  int* c = nullptr;
  if (give_up_counter(&c) != hipSuccess) return -1;
  if (hipDeviceSynchronize() != hipSuccess) return -1;
  int host = 0;
  if (hipMemcpy(&host, c, sizeof(int), hipMemcpyDeviceToHost) != hipSuccess) return -1;
  return host;
}

int dn_chunk_bwd_algo(const dn_chunk_bwd_args* a) {
  if (int rc = check_bwd(a)) return rc;
  return bwd_algo(a, bwd_dims(a));
}

size_t dn_chunk_bwd_workspace_bytes(const dn_chunk_bwd_args* a) {
  if (check_bwd(a)) return 0;
  const Dims d = bwd_dims(a);
  const int algo = bwd_algo(a, d);
  return algo < 0 ? 0 : bwd_workspace(run_dims(d, algo), algo, a->qkv_dtype);
}

int dn_chunk_bwd(const dn_chunk_bwd_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (int rc = check_bwd(a)) return rc;
  const int algo = bwd_algo(a, bwd_dims(a));
  if (algo < 0)
    return fail(DN_ERR_UNSUPPORTED, "DN_ALGO_MFMA needs bf16 q/k/v, head_k_dim 64 or 128 "
                                    "(or 256 with per-head gates and head_v_dim a multiple "
                                    "of 128), head_v_dim a multiple of 64, and chunk_len 64 "
                                    "with a per-channel forget gate");
  const Dims d = run_dims(bwd_dims(a), algo);
  const size_t need = bwd_workspace(d, algo, a->qkv_dtype);
  void* ws = a->workspace;
  if (ws) {
    if (a->workspace_bytes < need)
      return fail(DN_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) +
                                        " bytes");
  } else {
    hipError_t e = pool_get(need, &ws, stream);
    if (e != hipSuccess) return hip_fail(e, "workspace allocation");
  }
  const size_t nq = size_t(d.B) * d.S * d.H, ns = size_t(d.B) * d.H * d.K * d.V;
  if (a->check_finite) {
    std::vector<Guarded> in = {{a->d_y, nq * d.V, a->grad_dtype},
                               {a->d_state_final, ns, DN_F32},
                               {a->q, nq * d.K, a->qkv_dtype},
                               {a->k, nq * d.K, a->qkv_dtype},
                               {a->v, nq * d.V, a->qkv_dtype},
                               {a->erase, nq * d.ew, DN_F32},
                               {a->write, nq * d.ww, DN_F32},
                               {a->has_gate ? a->g : nullptr, nq * d.dw, DN_F32},
                               {a->state_in, ns, DN_F32}};
    if (int rc = nonfinite_check(in, stream, "inputs")) return rc;
  }
  hipError_t e;
  const float* g = a->has_gate ? a->g : nullptr;
  if (bwd_all_mfma(d, a->qkv_dtype, algo)) {
    char* base = static_cast<char*>(ws);
    float* states = reinterpret_cast<float*>(base);
    float* ds_after = reinterpret_cast<float*>(base + bwd_state_bytes(d));
    void* mws = base + 2 * bwd_state_bytes(d);
    const bool g4 = states_g4(d);
    e = mfma_bwd_scans(d, a->grad_dtype, a->d_y, a->d_state_final, a->q, a->k, a->v, a->erase,
                       a->write, g, a->state_in, states, ds_after, a->d_state, mws, stream, g4);
    if (e == hipSuccess)
      e = mfma_chunk_bwd(
          d, a->grad_dtype, a->d_y, a->q, a->k, a->v, a->erase, a->write, g, states, ds_after,
          a->d_q, a->d_k, a->d_v, a->d_erase, a->d_write, a->has_gate ? a->d_g : nullptr,
          mfma_bwd_tiles(d, mws),
          mfma_chunk_bwd_partials(d)
              ? reinterpret_cast<float*>(static_cast<char*>(mws) +
                                         align_up(mfma_bwd_workspace(d), 256))
              : nullptr,
          stream, g4);
  } else {
    e = generic_bwd(d, a->qkv_dtype, a->grad_dtype, a->d_y, a->d_state_final, a->q, a->k, a->v,
                    a->erase, a->write, g, a->state_in, a->d_q, a->d_k, a->d_v, a->d_erase,
                    a->d_write, a->has_gate ? a->d_g : nullptr, a->d_state, ws, stream,
                    algo == DN_ALGO_MFMA
                        ? static_cast<char*>(ws) + align_up(generic_bwd_workspace(d), 256)
                        : nullptr);
  }
  if (e != hipSuccess) return hip_fail(e, "dn_chunk_bwd launch");
  if (a->check_finite) {
    std::vector<Guarded> out = {{a->d_q, nq * d.K, a->grad_dtype},
                                {a->d_k, nq * d.K, a->grad_dtype},
                                {a->d_v, nq * d.V, a->grad_dtype},
                                {a->d_erase, nq * d.ew, DN_F32},
                                {a->d_write, nq * d.ww, DN_F32},
                                {a->has_gate ? a->d_g : nullptr, nq * d.dw, DN_F32},
                                {a->d_state, ns, DN_F32}};
    if (int rc = nonfinite_check(out, stream, "outputs")) return rc;
  }
  return DN_OK;
}

int dn_step(const dn_step_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  if (int rc = check_common(a->batch, 1, a->nheads, a->head_k_dim, a->head_v_dim,
                            a->erase_width, a->write_width, a->decay_width, a->has_gate))
    return rc;
  if (!valid_dtype(a->qkv_dtype) || !valid_dtype(a->y_dtype))
    return fail(DN_ERR_DTYPE, "dtype must be DN_F32 or DN_BF16");
  if (!a->q || !a->k || !a->v || !a->erase || !a->write || !a->state_in || !a->y ||
      !a->state_out || (a->has_gate && !a->g))
    return fail(DN_ERR_NULL, "a required tensor pointer is NULL");
  const size_t nh = size_t(a->batch) * a->nheads, ns = nh * a->head_k_dim * a->head_v_dim;
  if (a->check_finite) {
    std::vector<Guarded> in = {{a->q, nh * a->head_k_dim, a->qkv_dtype},
                               {a->k, nh * a->head_k_dim, a->qkv_dtype},
                               {a->v, nh * a->head_v_dim, a->qkv_dtype},
                               {a->erase, nh * a->erase_width, DN_F32},
                               {a->write, nh * a->write_width, DN_F32},
                               {a->has_gate ? a->g : nullptr, nh * a->decay_width, DN_F32},
                               {a->state_in, ns, DN_F32}};
    if (int rc = nonfinite_check(in, stream, "inputs")) return rc;
  }
  hipError_t e = launch_step(*a, resolve_scale(a->scale, a->head_k_dim), stream);
  if (e != hipSuccess) return hip_fail(e, "dn_step launch");
  if (a->check_finite) {
    std::vector<Guarded> out = {{a->y, nh * a->head_v_dim, a->y_dtype},
                                {a->state_out, ns, DN_F32}};
    if (int rc = nonfinite_check(out, stream, "outputs")) return rc;
  }
  return DN_OK;
}

namespace {

// dn_frontend's argument checks (also those of dn_frontend_chunk_fwd's `fe`).
int check_frontend(const dn_frontend_args* a) {
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  // conv.rs:88-90 and qkv.rs:397-401
  if (a->sequence < 1) return fail(DN_ERR_SEQUENCE, "sequence length must be at least 1");
  if (a->batch < 1 || a->nheads < 1 || a->head_k_dim < 1 || a->head_v_dim < 1 ||
      a->n_householder < 1 || a->conv_kernel < 0)
    return fail(DN_ERR_SHAPE, "batch, nheads, head_k_dim, head_v_dim and n_householder must be "
                              "at least 1, conv_kernel at least 0");
  if (a->head_k_dim > DN_FRONTEND_MAX_HEAD_DIM || a->head_v_dim > DN_FRONTEND_MAX_HEAD_DIM)
    return fail(DN_ERR_UNSUPPORTED, "dn_frontend supports head dims up to " +
                                        std::to_string(DN_FRONTEND_MAX_HEAD_DIM));
  if (a->conv_kernel > DN_FRONTEND_MAX_KERNEL)
    return fail(DN_ERR_UNSUPPORTED, "dn_frontend supports conv_kernel up to " +
                                        std::to_string(DN_FRONTEND_MAX_KERNEL));
  if (!valid_dtype(a->in_dtype) || !valid_dtype(a->out_dtype))
    return fail(DN_ERR_DTYPE, "dtype must be DN_F32 or DN_BF16");
  if (a->qk_norm == DN_QKNORM_SUM)
    return fail(DN_ERR_UNSUPPORTED, "QkNorm::Sum is not offered (its epsilon is burn_stack's)");
  if (a->qk_norm != DN_QKNORM_L2 && a->qk_norm != DN_QKNORM_NONE)
    return fail(DN_ERR_SHAPE, "unknown qk_norm");
  if (a->qk_activation < DN_ACT_IDENTITY || a->qk_activation > DN_ACT_ELU_PLUS_ONE)
    return fail(DN_ERR_SHAPE, "unknown qk_activation");
  if (a->conv_activation != DN_ACT_IDENTITY && a->conv_activation != DN_ACT_SILU)
    return fail(DN_ERR_SHAPE, "conv_activation must be DN_ACT_SILU or DN_ACT_IDENTITY");
  if (a->write_gate < DN_WRITE_FIXED || a->write_gate > DN_WRITE_CHANNEL)
    return fail(DN_ERR_SHAPE, "unknown write_gate");
  const bool has_conv = a->conv_kernel > 0;
  if (has_conv != (a->window_in != nullptr) || has_conv != (a->window_out != nullptr))
    return fail(DN_ERR_SHAPE, "convolution window presence must match the block's convolution");
  // Bounds the column arithmetic below (head dims are at most 4096).
  if (too_large({a->nheads, a->n_householder}, int64_t(1) << 31))
    return fail(DN_ERR_SHAPE, "tensor too large");
  const int64_t H = a->nheads, u = a->n_householder;
  const int64_t key_dim = H * a->head_k_dim, value_dim = H * a->head_v_dim;
  const int64_t conv_dim = key_dim + u * (key_dim + value_dim);
  const int64_t gate_w = a->write_gate == DN_WRITE_FIXED    ? 0
                         : a->write_gate == DN_WRITE_SCALAR ? u * H
                                                            : u * (key_dim + value_dim);
  if (a->proj_stride < conv_dim + gate_w)
    return fail(DN_ERR_SHAPE, "proj_stride " + std::to_string(a->proj_stride) +
                                  " is narrower than the conv and write-gate columns (" +
                                  std::to_string(conv_dim + gate_w) + ")");
  if (too_large({a->batch, a->sequence}, int64_t(1) << 31) || conv_dim >= (int64_t(1) << 31) ||
      too_large({a->batch, a->sequence, a->proj_stride}, int64_t(1) << 40) ||
      too_large({a->batch, a->sequence, gate_w > u * H ? gate_w : u * H}, int64_t(1) << 32))
    return fail(DN_ERR_SHAPE, "tensor too large");
  if (!a->projected || !a->q || !a->k || !a->v || !a->erase || !a->write ||
      (has_conv && !a->conv_weight))
    return fail(DN_ERR_NULL, "a required tensor pointer is NULL");
  if (a->write_gate == DN_WRITE_CHANNEL && a->write == a->erase)
    return fail(DN_ERR_SHAPE, "per-channel erase and write gates need separate buffers");
  return DN_OK;
}

// The front-end's outputs are the chunk forward's inputs, at the same sizes.
int check_frontend_chunk(const dn_frontend_chunk_fwd_args* a) {
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  if (int rc = check_frontend(&a->fe)) return rc;
  if (int rc = check_fwd(&a->fwd)) return rc;
  const dn_frontend_args& fe = a->fe;
  const dn_chunk_fwd_args& f = a->fwd;
  if (fe.n_householder != 1)
    return fail(DN_ERR_UNSUPPORTED,
                "dn_frontend_chunk_fwd takes n_householder 1 (DeltaProduct folds its micro-steps "
                "between dn_frontend and dn_chunk_fwd)");
  const bool ch = fe.write_gate == DN_WRITE_CHANNEL;
  if (fe.batch != f.batch || fe.sequence != f.sequence || fe.nheads != f.nheads ||
      fe.head_k_dim != f.head_k_dim || fe.head_v_dim != f.head_v_dim ||
      f.erase_width != (ch ? f.head_k_dim : 1) || f.write_width != (ch ? f.head_v_dim : 1) ||
      fe.out_dtype != f.qkv_dtype)
    return fail(DN_ERR_SHAPE, "the chunk forward's sizes, gate widths and dtype must be the "
                              "front-end's outputs'");
  if (f.q != fe.q || f.k != fe.k || f.v != fe.v || f.erase != fe.erase || f.write != fe.write)
    return fail(DN_ERR_SHAPE, "fwd.q, k, v, erase and write must be fe's outputs");
  return DN_OK;
}

// Where the front-end's q/k half runs in the intra kernel's load stage: the
// two-kernel MFMA forward with per-head gates at head_k_dim 128, a conv of
// length 4 with the reference's default activations (SiLU in the conv,
// nothing after it), bf16 throughout, and 16-byte rows.
bool fe_fusable(const dn_frontend_chunk_fwd_args* a, const Dims& d, int algo) {
  const dn_frontend_args& fe = a->fe;
  auto al = [](const void* p, size_t b) { return reinterpret_cast<uintptr_t>(p) % b == 0; };
  return algo == DN_ALGO_MFMA && !a->fwd.check_finite && d.K == 128 && d.ew == 1 &&
         d.ww == 1 && d.dw <= 1 && fe.conv_kernel == 4 && fe.conv_activation == DN_ACT_SILU &&
         fe.qk_activation == DN_ACT_SILU && fe.in_dtype == DN_BF16 &&
         fe.out_dtype == DN_BF16 && fe.proj_stride % 8 == 0 && al(fe.projected, 16) &&
         al(fe.conv_weight, 16) && al(fe.q, 16) && al(fe.k, 16);
}

}  // namespace

int dn_frontend(const dn_frontend_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (int rc = check_frontend(a)) return rc;
  hipError_t e = launch_frontend(*a, stream);
  if (e != hipSuccess) return hip_fail(e, "dn_frontend launch");
  return DN_OK;
}

size_t dn_frontend_chunk_fwd_workspace_bytes(const dn_frontend_chunk_fwd_args* a) {
  if (check_frontend_chunk(a)) return 0;
  return dn_chunk_fwd_workspace_bytes(&a->fwd);
}

int dn_frontend_chunk_fwd(const dn_frontend_chunk_fwd_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (int rc = check_frontend_chunk(a)) return rc;
  const dn_frontend_args& fe = a->fe;
  const dn_chunk_fwd_args* f = &a->fwd;
  Dims d = make_dims(f->batch, f->sequence, f->nheads, f->head_k_dim, f->head_v_dim,
                     f->erase_width, f->write_width, f->decay_width, f->has_gate, f->chunk_len,
                     f->scale);
  const int algo = fwd_algo(f, d);
  if (algo < 0)
    return fail(DN_ERR_UNSUPPORTED, "the requested MFMA path does not cover this shape/dtype");
  if (!fe_fusable(a, run_dims(d, algo), algo)) {
    // The two calls in turn.
    if (int rc = dn_frontend(&fe, stream)) return rc;
    return dn_chunk_fwd(f, stream);
  }
  d = run_dims(d, algo);
  const size_t need = fwd_workspace(d, algo);
  void* ws = f->workspace;
  if (ws) {
    if (f->workspace_bytes < need)
      return fail(DN_ERR_WORKSPACE, "workspace too small: need " + std::to_string(need) +
                                        " bytes");
  } else if (need) {
    hipError_t e = pool_get(need, &ws, stream);
    if (e != hipSuccess) return hip_fail(e, "workspace allocation");
  }
  // v and the write gates; then q and k in the intra kernel, which reads the
  // old conv window; then the next window.
  hipError_t e = launch_frontend(fe, stream, kFrontV | kFrontGates);
  if (e != hipSuccess) return hip_fail(e, "dn_frontend_chunk_fwd front-end launch");
  FeParams fp{};
  fp.proj = static_cast<const uint16_t*>(fe.projected);
  fp.stride = fe.proj_stride;
  fp.w = fe.conv_weight;
  fp.bias = fe.conv_bias;
  fp.win = static_cast<const uint16_t*>(fe.window_in);
  fp.conv_dim = int(fe.nheads * (2 * fe.head_k_dim + fe.head_v_dim));
  fp.l2 = fe.qk_norm == DN_QKNORM_L2;
  fp.q = static_cast<uint16_t*>(fe.q);
  fp.k = static_cast<uint16_t*>(fe.k);
  e = mfma_fwd(d, f->y_dtype, f->q, f->k, f->v, f->erase, f->write,
               f->has_gate ? f->g : nullptr, f->state_in, f->y, f->state_out, ws, stream, false,
               &fp);
  if (e != hipSuccess) return hip_fail(e, "dn_frontend_chunk_fwd launch");
  e = launch_frontend(fe, stream, kFrontWindow);
  if (e != hipSuccess) return hip_fail(e, "dn_frontend_chunk_fwd window launch");
  return DN_OK;
}

int dn_out_norm(const dn_out_norm_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  if (a->tokens < 1 || a->nheads < 1 || a->head_v_dim < 1)
    return fail(DN_ERR_SHAPE, "tokens, nheads and head_v_dim must be at least 1");
  if (a->head_v_dim > DN_OUT_NORM_MAX_HEAD_DIM)
    return fail(DN_ERR_UNSUPPORTED, "dn_out_norm supports head_v_dim up to " +
                                        std::to_string(DN_OUT_NORM_MAX_HEAD_DIM));
  if (!valid_dtype(a->x_dtype) || !valid_dtype(a->out_dtype) ||
      (a->gate && !valid_dtype(a->gate_dtype)))
    return fail(DN_ERR_DTYPE, "dtype must be DN_F32 or DN_BF16");
  if (!a->x || !a->weight || !a->out) return fail(DN_ERR_NULL, "a required tensor pointer is NULL");
  if (a->gate && a->gate_stride < a->nheads * a->head_v_dim)
    return fail(DN_ERR_SHAPE, "gate_stride is narrower than one token's gates");
  if (!(a->eps >= 0.0)) return fail(DN_ERR_SHAPE, "eps must be a non-negative number");
  if (too_large({a->tokens, a->nheads}, int64_t(1) << 40))
    return fail(DN_ERR_SHAPE, "tensor too large");
  hipError_t e = launch_out_norm(*a, stream);
  if (e != hipSuccess) return hip_fail(e, "dn_out_norm launch");
  return DN_OK;
}

int dn_block_step(const dn_block_step_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  if (a->batch < 1 || a->nheads < 1 || a->head_k_dim < 1 || a->head_v_dim < 1 ||
      a->conv_kernel < 0)
    return fail(DN_ERR_SHAPE, "batch, nheads, head_k_dim and head_v_dim must be at least 1, "
                              "conv_kernel at least 0");
  if (a->head_k_dim > DN_BLOCK_STEP_MAX_HEAD_DIM || a->head_v_dim > DN_BLOCK_STEP_MAX_HEAD_DIM)
    return fail(DN_ERR_UNSUPPORTED, "dn_block_step supports head dims up to " +
                                        std::to_string(DN_BLOCK_STEP_MAX_HEAD_DIM));
  if (a->head_v_dim % block_step_cols(a->head_v_dim))
    return fail(DN_ERR_UNSUPPORTED, "dn_block_step needs head_v_dim even above 64 and a "
                                    "multiple of 4 above 128");
  if (a->conv_kernel > DN_FRONTEND_MAX_KERNEL)
    return fail(DN_ERR_UNSUPPORTED, "dn_block_step supports conv_kernel up to " +
                                        std::to_string(DN_FRONTEND_MAX_KERNEL));
  if (!valid_dtype(a->in_dtype) || !valid_dtype(a->out_dtype))
    return fail(DN_ERR_DTYPE, "dtype must be DN_F32 or DN_BF16");
  if (a->qk_norm == DN_QKNORM_SUM)
    return fail(DN_ERR_UNSUPPORTED, "QkNorm::Sum is not offered (its epsilon is burn_stack's)");
  if (a->qk_norm != DN_QKNORM_L2 && a->qk_norm != DN_QKNORM_NONE)
    return fail(DN_ERR_SHAPE, "unknown qk_norm");
  if (a->qk_activation < DN_ACT_IDENTITY || a->qk_activation > DN_ACT_ELU_PLUS_ONE)
    return fail(DN_ERR_SHAPE, "unknown qk_activation");
  if (a->conv_activation != DN_ACT_IDENTITY && a->conv_activation != DN_ACT_SILU)
    return fail(DN_ERR_SHAPE, "conv_activation must be DN_ACT_SILU or DN_ACT_IDENTITY");
  if (a->write_gate < DN_WRITE_FIXED || a->write_gate > DN_WRITE_CHANNEL)
    return fail(DN_ERR_SHAPE, "unknown write_gate");
  if (a->has_gate && a->decay_width != 1 && a->decay_width != a->head_k_dim)
    return fail(DN_ERR_GATE_WIDTH, "forget gate: last axis must be 1 or " +
                                       std::to_string(a->head_k_dim) + ", got " +
                                       std::to_string(a->decay_width));
  if (!(a->eps >= 0.0)) return fail(DN_ERR_SHAPE, "eps must be a non-negative number");
  const bool has_conv = a->conv_kernel > 0;
  if (has_conv != (a->window_in != nullptr) || has_conv != (a->window_out != nullptr))
    return fail(DN_ERR_SHAPE, "convolution window presence must match the block's convolution");
  if (a->nheads > INT32_MAX) return fail(DN_ERR_SHAPE, "tensor too large");
  const int64_t H = a->nheads, key_dim = H * a->head_k_dim, value_dim = H * a->head_v_dim;
  const int64_t conv_dim = 2 * key_dim + value_dim;
  const int64_t gate_w = a->write_gate == DN_WRITE_FIXED    ? 0
                         : a->write_gate == DN_WRITE_SCALAR ? H
                                                            : key_dim + value_dim;
  const int64_t width = conv_dim + gate_w + (a->norm_gated ? value_dim : 0);
  if (a->proj_stride < width)
    return fail(DN_ERR_SHAPE, "proj_stride " + std::to_string(a->proj_stride) +
                                  " is narrower than the conv, write-gate and norm-gate columns (" +
                                  std::to_string(width) + ")");
  if (too_large({a->batch, H}, int64_t(1) << 31) ||
      too_large({a->batch, a->proj_stride}, int64_t(1) << 40))
    return fail(DN_ERR_SHAPE, "tensor too large");
  if (!a->projected || !a->state_in || !a->state_out || !a->norm_weight || !a->out ||
      (has_conv && !a->conv_weight) || (a->has_gate && !a->g))
    return fail(DN_ERR_NULL, "a required tensor pointer is NULL");
  const int C = block_step_cols(a->head_v_dim);
  if ((reinterpret_cast<uintptr_t>(a->state_in) | reinterpret_cast<uintptr_t>(a->state_out)) %
      (4 * C))
    return fail(DN_ERR_UNSUPPORTED, "dn_block_step needs the state aligned to " +
                                        std::to_string(4 * C) + " bytes");
  const size_t ns = size_t(a->batch) * H * a->head_k_dim * a->head_v_dim;
  const size_t nw = has_conv ? size_t(a->batch) * conv_dim * a->conv_kernel : 0;
  if (a->check_finite) {
    std::vector<Guarded> in = {{a->projected, size_t(a->batch) * a->proj_stride, a->in_dtype},
                               {a->window_in, nw, a->in_dtype},
                               {a->has_gate ? a->g : nullptr, size_t(a->batch) * H * a->decay_width,
                                DN_F32},
                               {a->state_in, ns, DN_F32}};
    if (int rc = nonfinite_check(in, stream, "inputs")) return rc;
  }
  hipError_t e = launch_block_step(*a, resolve_scale(a->scale, a->head_k_dim), stream);
  if (e != hipSuccess) return hip_fail(e, "dn_block_step launch");
  if (a->check_finite) {
    std::vector<Guarded> out = {{a->out, size_t(a->batch) * value_dim, a->out_dtype},
                                {a->window_out, nw, a->in_dtype},
                                {a->state_out, ns, DN_F32}};
    if (int rc = nonfinite_check(out, stream, "outputs")) return rc;
  }
  return DN_OK;
}

int dn_unit_lower_inverse(const dn_tri_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  if (a->batch < 0 || a->size < 0) return fail(DN_ERR_SHAPE, "batch and size must be at least 0");
  if (a->size > (int64_t(1) << 20) || too_large({a->batch, a->size, a->size}, int64_t(1) << 40) ||
      too_large({a->batch, (a->size + 63) / 64}, int64_t(1) << 31))
    return fail(DN_ERR_SHAPE, "tensor too large");
  if (a->solve != DN_TRI_BLOCKED && a->solve != DN_TRI_NEUMANN)
    return fail(DN_ERR_UNSUPPORTED, "solve must be DN_TRI_BLOCKED or DN_TRI_NEUMANN");
  if (a->solve == DN_TRI_NEUMANN && a->size > DN_TRI_NEUMANN_MAX_SIZE)
    return fail(DN_ERR_UNSUPPORTED, "DN_TRI_NEUMANN supports size up to " +
                                        std::to_string(DN_TRI_NEUMANN_MAX_SIZE) +
                                        "; DN_TRI_BLOCKED covers any size");
  const size_t nm = size_t(a->batch) * a->size * a->size;
  if (nm == 0) return DN_OK;
  if (!a->n_strict || !a->t) return fail(DN_ERR_NULL, "a required tensor pointer is NULL");
  if (a->check_finite) {
    if (int rc = nonfinite_check({{a->n_strict, nm, DN_F32}}, stream, "inputs")) return rc;
  }
  hipError_t e = launch_unit_lower_inverse(*a, stream);
  if (e != hipSuccess) return hip_fail(e, "dn_unit_lower_inverse launch");
  if (a->check_finite) {
    if (int rc = nonfinite_check({{a->t, nm, DN_F32}}, stream, "outputs")) return rc;
  }
  return DN_OK;
}

int dn_recurrent(const dn_recurrent_args* a, hipStream_t stream) {
  g_last_error.clear();
  if (!a) return fail(DN_ERR_NULL, "args is NULL");
  if (int rc = check_common(a->batch, a->sequence, a->nheads, a->head_k_dim, a->head_v_dim,
                            a->erase_width, a->write_width, a->decay_width, a->has_gate))
    return rc;
  if (!valid_dtype(a->qkv_dtype) || !valid_dtype(a->y_dtype))
    return fail(DN_ERR_DTYPE, "dtype must be DN_F32 or DN_BF16");
  if (!a->q || !a->k || !a->v || !a->erase || !a->write || !a->state_in || !a->y ||
      !a->state_out || (a->has_gate && !a->g))
    return fail(DN_ERR_NULL, "a required tensor pointer is NULL");
  if (!recurrent_supported(*a))
    return fail(DN_ERR_UNSUPPORTED, "dn_recurrent supports head_k_dim up to " +
                                        std::to_string(kRecMaxK) +
                                        "; run dn_step per token for larger heads");
  const size_t nq = size_t(a->batch) * a->sequence * a->nheads;
  const size_t ns = size_t(a->batch) * a->nheads * a->head_k_dim * a->head_v_dim;
  if (a->check_finite) {
    std::vector<Guarded> in = {{a->q, nq * a->head_k_dim, a->qkv_dtype},
                               {a->k, nq * a->head_k_dim, a->qkv_dtype},
                               {a->v, nq * a->head_v_dim, a->qkv_dtype},
                               {a->erase, nq * a->erase_width, DN_F32},
                               {a->write, nq * a->write_width, DN_F32},
                               {a->has_gate ? a->g : nullptr, nq * a->decay_width, DN_F32},
                               {a->state_in, ns, DN_F32}};
    if (int rc = nonfinite_check(in, stream, "inputs")) return rc;
  }
  hipError_t e = launch_recurrent(*a, resolve_scale(a->scale, a->head_k_dim), stream);
  if (e != hipSuccess) return hip_fail(e, "dn_recurrent launch");
  if (a->check_finite) {
    std::vector<Guarded> out = {{a->y, nq * a->head_v_dim, a->y_dtype},
                                {a->state_out, ns, DN_F32}};
    if (int rc = nonfinite_check(out, stream, "outputs")) return rc;
  }
  return DN_OK;
}

}  // extern "C"
