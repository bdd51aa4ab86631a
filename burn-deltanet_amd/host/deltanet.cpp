// Host-side C++ mirror of burn-deltanet's delta-rule core interface, over the
// C ABI of deltanet_core.h. Declarations and the reference each function
// mirrors are in deltanet.hpp. No device code: every computation is a
// dn_chunk_fwd / dn_step / dn_chunk_bwd call; this layer checks shapes with
// the reference's messages, allocates the fresh output tensors the
// reference's functional interface returns, and lays out the per-token
// slices of the recurrent path.

#include "deltanet.hpp"

#include <hip/hip_runtime_api.h>

#include <algorithm>
#include <cmath>
#include <limits>
#include <memory>
#include <vector>
#include <sstream>

namespace deltanet {
namespace {

std::string shape_str(const std::vector<int64_t>& d) {
  std::ostringstream o;
  o << "[";
  for (size_t i = 0; i < d.size(); ++i) o << (i ? ", " : "") << d[i];
  o << "]";
  return o.str();
}

void expect_shape(const Tensor& t, const std::vector<int64_t>& shape, const char* what) {
  if (t.dims() != shape)
    throw Error(DN_ERR_SHAPE, std::string(what) + ": expected shape " + shape_str(shape) +
                                  ", got " + shape_str(t.dims()));
}

// A gate axis is either shared across the head (width 1) or per channel
// (path.rs:186-197).
void gate_axis(const Tensor& t, const std::vector<int64_t>& lead, int64_t full, const char* what) {
  const auto& d = t.dims();
  if (d.size() != lead.size() + 1 || !std::equal(lead.begin(), lead.end(), d.begin()))
    throw Error(DN_ERR_SHAPE, std::string(what) + ": expected leading dims " + shape_str(lead) +
                                  ", got " + shape_str(d));
  if (d.back() != 1 && d.back() != full)
    throw Error(DN_ERR_GATE_WIDTH, std::string(what) + ": last axis must be 1 or " +
                                       std::to_string(full) + ", got " + std::to_string(d.back()));
}

void require_defined(const Tensor& t, const char* what) {
  if (!t.defined()) throw Error(DN_ERR_NULL, std::string(what) + ": tensor is not defined");
}

void require_f32(const Tensor& t, const char* what) {
  if (t.dtype() != DType::F32)
    throw Error(DN_ERR_DTYPE, std::string(what) + ": gates and state must be float32");
}

DType qkv_dtype(const Tensor& q, const Tensor& k, const Tensor& v) {
  if (q.dtype() != k.dtype() || q.dtype() != v.dtype())
    throw Error(DN_ERR_DTYPE, "q, k and v must share one dtype");
  return q.dtype();
}

void check(int rc) {
  if (rc != DN_OK) throw Error(rc, dn_last_error());
}

void check_hip(hipError_t e, const char* what) {
  if (e != hipSuccess)
    throw Error(DN_ERR_HIP, std::string(what) + ": " + hipGetErrorString(e));
}

double nan_scale(const std::optional<double>& s) {
  return s ? *s : std::numeric_limits<double>::quiet_NaN();
}

// The calling thread's Workspace on the current device (the default of the
// functions that take a Workspace*).
Workspace& thread_workspace() {
  thread_local std::vector<std::unique_ptr<Workspace>> per_device;
  int dev = 0;
  check_hip(hipGetDevice(&dev), "hipGetDevice");
  if (size_t(dev) >= per_device.size()) per_device.resize(size_t(dev) + 1);
  if (!per_device[size_t(dev)]) per_device[size_t(dev)] = std::make_unique<Workspace>();
  return *per_device[size_t(dev)];
}

}  // namespace

Workspace::~Workspace() {
  if (ptr_) (void)hipFree(ptr_);
}

void* Workspace::reserve(size_t bytes, hipStream_t stream) {
  if (bytes <= bytes_) return ptr_;
  if (ptr_) check_hip(hipFreeAsync(ptr_, stream), "hipFreeAsync");
  ptr_ = nullptr;
  bytes_ = 0;
  check_hip(hipMallocAsync(&ptr_, bytes, stream), "hipMallocAsync");
  bytes_ = bytes;
  return ptr_;
}

Error::Error(int status, const std::string& what) : std::runtime_error(what), status_(status) {}

size_t dtype_size(DType dtype) { return dtype == DType::BF16 ? 2 : 4; }

size_t Tensor::numel() const {
  size_t n = 1;
  for (int64_t d : dims_) n *= size_t(d);
  return dims_.empty() ? 0 : n;
}

Tensor Tensor::empty(std::vector<int64_t> dims, DType dtype) {
  Tensor t;
  t.dims_ = std::move(dims);
  t.dtype_ = dtype;
  void* p = nullptr;
  const size_t bytes = t.bytes();
  check_hip(hipMalloc(&p, bytes ? bytes : 1), "hipMalloc");
  t.owner_ = std::shared_ptr<void>(p, [](void* q) { (void)hipFree(q); });
  t.data_ = p;
  return t;
}

Tensor Tensor::view(void* data, std::vector<int64_t> dims, DType dtype) {
  Tensor t;
  t.data_ = data;
  t.dims_ = std::move(dims);
  t.dtype_ = dtype;
  return t;
}

Tensor Tensor::reshape(std::vector<int64_t> dims) const {
  Tensor t = *this;
  t.dims_ = std::move(dims);
  if (t.numel() != numel())
    throw Error(DN_ERR_SHAPE, "reshape: " + shape_str(dims_) + " to " + shape_str(t.dims_) +
                                  " changes the element count");
  return t;
}

std::pair<Tensor, Tensor> beta_gates(const Tensor& beta) {
  std::vector<int64_t> d = beta.dims();
  d.push_back(1);
  Tensor g = beta.reshape(d);
  return {g, g};
}

// ---------------------------------------------------------------------------
// DeltaInput (path.rs:143-231)
// ---------------------------------------------------------------------------
DeltaInput::Dims DeltaInput::dims() const {
  if (q_bshk.rank() != 4 || v_bshv.rank() != 4)
    throw Error(DN_ERR_SHAPE, "q and v must be [batch, sequence, nheads, head_dim]");
  return Dims{q_bshk.dim(0), q_bshk.dim(1), q_bshk.dim(2), q_bshk.dim(3), v_bshv.dim(3)};
}

double DeltaInput::resolved_scale() const {
  return scale ? *scale : 1.0 / std::sqrt(double(dims().head_k_dim));
}

bool DeltaInput::has_channel_decay() const { return g_bshK && g_bshK->dim(3) > 1; }

void DeltaInput::sanity() const {
  require_defined(q_bshk, "q");
  require_defined(k_bshk, "k");
  require_defined(v_bshv, "v");
  require_defined(erase_bshK, "erase gate");
  require_defined(write_bshV, "write gate");
  require_defined(state_bhkv, "state");
  const Dims d = dims();
  if (d.sequence <= 0) throw Error(DN_ERR_SEQUENCE, "sequence length must be at least 1");
  expect_shape(k_bshk, {d.batch, d.sequence, d.nheads, d.head_k_dim}, "k");
  expect_shape(v_bshv, {d.batch, d.sequence, d.nheads, d.head_v_dim}, "v");
  expect_shape(state_bhkv, {d.batch, d.nheads, d.head_k_dim, d.head_v_dim}, "state");
  gate_axis(erase_bshK, {d.batch, d.sequence, d.nheads}, d.head_k_dim, "erase gate");
  gate_axis(write_bshV, {d.batch, d.sequence, d.nheads}, d.head_v_dim, "write gate");
  if (g_bshK) {
    require_defined(*g_bshK, "forget gate");
    gate_axis(*g_bshK, {d.batch, d.sequence, d.nheads}, d.head_k_dim, "forget gate");
  }
  qkv_dtype(q_bshk, k_bshk, v_bshv);
  require_f32(erase_bshK, "erase gate");
  require_f32(write_bshV, "write gate");
  require_f32(state_bhkv, "state");
  if (g_bshK) require_f32(*g_bshK, "forget gate");
}

std::pair<Tensor, Tensor> DeltaInput::run(const DeltaPath& path, hipStream_t stream,
                                          bool check_finite, Workspace* ws) const {
  sanity();
  if (path.kind == DeltaPath::Kind::Recurrent) return delta_recurrent(stream, check_finite);
  const int64_t chunk_len = path.chunk_len.value_or(DeltaPath::DEFAULT_CHUNK_LEN);
  if (chunk_len <= 0) throw Error(DN_ERR_CHUNK_LEN, "chunk_len must be at least 1");
  // Chunk and ChunkRecalculated compute identical values; they differ only in
  // what a tape keeps, and this forward keeps nothing.
  return delta_chunk_recalculated(chunk_len, stream, check_finite, ws);
}

std::pair<Tensor, Tensor> DeltaInput::delta_chunk_recalculated(int64_t chunk_len,
                                                               hipStream_t stream,
                                                               bool check_finite,
                                                               Workspace* ws) const {
  sanity();
  if (chunk_len <= 0) throw Error(DN_ERR_CHUNK_LEN, "chunk_len must be at least 1");
  if (chunk_len > std::numeric_limits<int32_t>::max())
    throw Error(DN_ERR_CHUNK_LEN, "chunk_len must fit in 32 bits");
  const Dims d = dims();
  const DType dt = q_bshk.dtype();
  Tensor y = Tensor::empty({d.batch, d.sequence, d.nheads, d.head_v_dim}, dt);
  Tensor s = Tensor::empty({d.batch, d.nheads, d.head_k_dim, d.head_v_dim}, DType::F32);
  dn_chunk_fwd_args a{};
  a.batch = d.batch;
  a.sequence = d.sequence;
  a.nheads = d.nheads;
  a.head_k_dim = d.head_k_dim;
  a.head_v_dim = d.head_v_dim;
  a.erase_width = erase_bshK.dim(3);
  a.write_width = write_bshV.dim(3);
  a.decay_width = g_bshK ? g_bshK->dim(3) : 0;
  a.has_gate = g_bshK ? 1 : 0;
  a.chunk_len = int32_t(chunk_len);
  a.scale = nan_scale(scale);
  a.qkv_dtype = int32_t(dt);
  a.y_dtype = int32_t(dt);
  a.algo = DN_ALGO_AUTO;
  a.check_finite = check_finite ? 1 : 0;
  a.q = q_bshk.data();
  a.k = k_bshk.data();
  a.v = v_bshv.data();
  a.erase = static_cast<const float*>(erase_bshK.data());
  a.write = static_cast<const float*>(write_bshV.data());
  a.g = g_bshK ? static_cast<const float*>(g_bshK->data()) : nullptr;
  a.state_in = static_cast<const float*>(state_bhkv.data());
  a.y = y.data();
  a.state_out = static_cast<float*>(s.data());
  // The workspace is this mirror's (the caller's, or the thread's own), never
  // the library's shared pool.
  const size_t need = dn_chunk_fwd_workspace_bytes(&a);
  if (need) {
    a.workspace = (ws ? *ws : thread_workspace()).reserve(need, stream);
    a.workspace_bytes = need;
  }
  check(dn_chunk_fwd(&a, stream));
  return {y, s};
}

std::pair<Tensor, Tensor> DeltaInput::delta_recurrent(hipStream_t stream,
                                                      bool check_finite) const {
  sanity();
  const Dims d = dims();
  const DType dt = q_bshk.dtype();
  const double sc = resolved_scale();
  Tensor y = Tensor::empty({d.batch, d.sequence, d.nheads, d.head_v_dim}, dt);
  if (d.head_k_dim <= DN_RECURRENT_MAX_K) {
    // One dn_recurrent call: the state stays on chip across the tokens.
    Tensor s = Tensor::empty(state_bhkv.dims(), DType::F32);
    dn_recurrent_args a{};
    a.batch = d.batch;
    a.sequence = d.sequence;
    a.nheads = d.nheads;
    a.head_k_dim = d.head_k_dim;
    a.head_v_dim = d.head_v_dim;
    a.erase_width = erase_bshK.dim(3);
    a.write_width = write_bshV.dim(3);
    a.decay_width = g_bshK ? g_bshK->dim(3) : 0;
    a.has_gate = g_bshK ? 1 : 0;
    a.scale = sc;
    a.qkv_dtype = int32_t(dt);
    a.y_dtype = int32_t(dt);
    a.check_finite = check_finite ? 1 : 0;
    a.q = q_bshk.data();
    a.k = k_bshk.data();
    a.v = v_bshv.data();
    a.erase = static_cast<const float*>(erase_bshK.data());
    a.write = static_cast<const float*>(write_bshV.data());
    a.g = g_bshK ? static_cast<const float*>(g_bshK->data()) : nullptr;
    a.state_in = static_cast<const float*>(state_bhkv.data());
    a.y = y.data();
    a.state_out = static_cast<float*>(s.data());
    check(dn_recurrent(&a, stream));
    return {y, s};
  }
  // head_k_dim above dn_recurrent's limit: dn_step per token, in place.
  Tensor state = Tensor::empty(state_bhkv.dims(), DType::F32);
  check_hip(hipMemcpyAsync(state.data(), state_bhkv.data(), state.bytes(),
                           hipMemcpyDeviceToDevice, stream),
            "hipMemcpyAsync");
  // Per-token slices [batch, nheads, ·] of the [batch, sequence, nheads, ·]
  // inputs: rows of nheads·width elements, sequence·nheads·width apart.
  auto slice_buf = [&](const Tensor& x) {
    return Tensor::empty({d.batch, d.nheads, x.dim(3)}, x.dtype());
  };
  Tensor qt = slice_buf(q_bshk), kt = slice_buf(k_bshk), vt = slice_buf(v_bshv);
  Tensor et = slice_buf(erase_bshK), wt = slice_buf(write_bshV);
  std::optional<Tensor> gt;
  if (g_bshK) gt = slice_buf(*g_bshK);
  Tensor yt = Tensor::empty({d.batch, d.nheads, d.head_v_dim}, dt);
  auto gather = [&](Tensor& dst, const Tensor& src, int64_t t) {
    const size_t row = size_t(d.nheads * src.dim(3)) * dtype_size(src.dtype());
    const char* from = static_cast<const char*>(src.data()) + size_t(t) * row;
    check_hip(hipMemcpy2DAsync(dst.data(), row, from, row * size_t(d.sequence), row,
                               size_t(d.batch), hipMemcpyDeviceToDevice, stream),
              "hipMemcpy2DAsync");
  };
  for (int64_t t = 0; t < d.sequence; ++t) {
    gather(qt, q_bshk, t);
    gather(kt, k_bshk, t);
    gather(vt, v_bshv, t);
    gather(et, erase_bshK, t);
    gather(wt, write_bshV, t);
    if (gt) gather(*gt, *g_bshK, t);
    delta_step_in_place(qt, kt, vt, et, wt, gt, state, yt, sc, stream, check_finite);
    const size_t row = size_t(d.nheads * d.head_v_dim) * dtype_size(dt);
    check_hip(hipMemcpy2DAsync(static_cast<char*>(y.data()) + size_t(t) * row,
                               row * size_t(d.sequence), yt.data(), row, row, size_t(d.batch),
                               hipMemcpyDeviceToDevice, stream),
              "hipMemcpy2DAsync");
  }
  // The slices are freed when this returns: finish with them first.
  check_hip(hipStreamSynchronize(stream), "hipStreamSynchronize");
  return {y, state};
}

// ---------------------------------------------------------------------------
// delta_step (recurrent.rs:41-99)
// ---------------------------------------------------------------------------
namespace {

dn_step_args step_args(const Tensor& q, const Tensor& k, const Tensor& v, const Tensor& e,
                       const Tensor& w, const std::optional<Tensor>& g, const Tensor& state,
                       double scale, bool check_finite) {
  require_defined(q, "q");
  require_defined(k, "k");
  require_defined(v, "v");
  require_defined(e, "erase gate");
  require_defined(w, "write gate");
  require_defined(state, "state");
  if (q.rank() != 3 || v.rank() != 3)
    throw Error(DN_ERR_SHAPE, "q and v must be [batch, nheads, head_dim]");
  const int64_t batch = q.dim(0), nheads = q.dim(1), hk = q.dim(2), hv = v.dim(2);
  expect_shape(k, {batch, nheads, hk}, "k");
  expect_shape(state, {batch, nheads, hk, hv}, "state");
  gate_axis(e, {batch, nheads}, hk, "erase gate");
  gate_axis(w, {batch, nheads}, hv, "write gate");
  if (g) gate_axis(*g, {batch, nheads}, hk, "forget gate");
  const DType dt = qkv_dtype(q, k, v);
  require_f32(e, "erase gate");
  require_f32(w, "write gate");
  require_f32(state, "state");
  if (g) require_f32(*g, "forget gate");
  dn_step_args a{};
  a.batch = batch;
  a.nheads = nheads;
  a.head_k_dim = hk;
  a.head_v_dim = hv;
  a.erase_width = e.dim(2);
  a.write_width = w.dim(2);
  a.decay_width = g ? g->dim(2) : 0;
  a.has_gate = g ? 1 : 0;
  a.scale = scale;
  a.qkv_dtype = int32_t(dt);
  a.y_dtype = int32_t(dt);
  a.check_finite = check_finite ? 1 : 0;
  a.q = q.data();
  a.k = k.data();
  a.v = v.data();
  a.erase = static_cast<const float*>(e.data());
  a.write = static_cast<const float*>(w.data());
  a.g = g ? static_cast<const float*>(g->data()) : nullptr;
  a.state_in = static_cast<const float*>(state.data());
  return a;
}

}  // namespace

Tensor unit_lower_inverse(const Tensor& n_strict, TriSolve solve, hipStream_t stream,
                          bool check_finite) {
  const int r = n_strict.rank();
  if (r < 2 || n_strict.dim(r - 2) != n_strict.dim(r - 1))
    throw Error(DN_ERR_SHAPE, "unit_lower_inverse expects a square trailing block");
  if (n_strict.dtype() != DType::F32)
    throw Error(DN_ERR_DTYPE, "unit_lower_inverse: n_strict must be float32");
  const int64_t size = n_strict.dim(r - 1);
  Tensor t = Tensor::empty(n_strict.dims(), DType::F32);
  if (n_strict.numel() == 0) return t;
  require_defined(n_strict, "n_strict");
  dn_tri_args a{};
  a.batch = int64_t(n_strict.numel()) / (size * size);
  a.size = size;
  a.solve = solve == TriSolve::Neumann ? DN_TRI_NEUMANN : DN_TRI_BLOCKED;
  a.check_finite = check_finite ? 1 : 0;
  a.n_strict = static_cast<const float*>(n_strict.data());
  a.t = static_cast<float*>(t.data());
  check(dn_unit_lower_inverse(&a, stream));
  return t;
}

std::pair<Tensor, Tensor> delta_step(const Tensor& q_bhk, const Tensor& k_bhk, const Tensor& v_bhv,
                                     const Tensor& erase_bhK, const Tensor& write_bhV,
                                     const std::optional<Tensor>& g_bhK, const Tensor& state_bhkv,
                                     double scale, hipStream_t stream, bool check_finite) {
  dn_step_args a = step_args(q_bhk, k_bhk, v_bhv, erase_bhK, write_bhV, g_bhK, state_bhkv, scale,
                             check_finite);
  Tensor y = Tensor::empty({a.batch, a.nheads, a.head_v_dim}, q_bhk.dtype());
  Tensor s = Tensor::empty(state_bhkv.dims(), DType::F32);
  a.y = y.data();
  a.state_out = static_cast<float*>(s.data());
  check(dn_step(&a, stream));
  return {y, s};
}

void delta_step_in_place(const Tensor& q_bhk, const Tensor& k_bhk, const Tensor& v_bhv,
                         const Tensor& erase_bhK, const Tensor& write_bhV,
                         const std::optional<Tensor>& g_bhK, Tensor& state_bhkv, Tensor& y_bhv,
                         double scale, hipStream_t stream, bool check_finite) {
  dn_step_args a = step_args(q_bhk, k_bhk, v_bhv, erase_bhK, write_bhV, g_bhK, state_bhkv, scale,
                             check_finite);
  require_defined(y_bhv, "y");
  expect_shape(y_bhv, {a.batch, a.nheads, a.head_v_dim}, "y");
  if (y_bhv.dtype() != q_bhk.dtype()) throw Error(DN_ERR_DTYPE, "y: dtype must match q");
  a.y = y_bhv.data();
  a.state_out = static_cast<float*>(state_bhkv.data());
  check(dn_step(&a, stream));
}

// ---------------------------------------------------------------------------
// combined_backward (combined_backward.rs:72-189)
// ---------------------------------------------------------------------------
DeltaChunkGrads combined_backward(const Tensor& d_y_bshv,
                                  const std::optional<Tensor>& d_final_state_bhkv,
                                  const Tensor& q_bshk, const Tensor& k_bshk, const Tensor& v_bshv,
                                  const Tensor& erase_bshK, const Tensor& write_bshV,
                                  const std::optional<Tensor>& g_bshK, const Tensor& state_bhkv,
                                  int64_t chunk_len, double scale, hipStream_t stream,
                                  bool check_finite, Workspace* ws) {
  DeltaInput in{q_bshk, k_bshk, v_bshv, erase_bshK, write_bshV, g_bshK, state_bhkv, scale};
  in.sanity();
  if (chunk_len <= 0) throw Error(DN_ERR_CHUNK_LEN, "chunk_len must be at least 1");
  if (chunk_len > std::numeric_limits<int32_t>::max())
    throw Error(DN_ERR_CHUNK_LEN, "chunk_len must fit in 32 bits");
  const DeltaInput::Dims d = in.dims();
  require_defined(d_y_bshv, "d_y");
  expect_shape(d_y_bshv, {d.batch, d.sequence, d.nheads, d.head_v_dim}, "d_y");
  if (d_final_state_bhkv) {
    expect_shape(*d_final_state_bhkv, state_bhkv.dims(), "d_final_state");
    require_f32(*d_final_state_bhkv, "d_final_state");
  }
  const DType gdt = d_y_bshv.dtype();
  DeltaChunkGrads g;
  g.d_q_bshk = Tensor::empty(q_bshk.dims(), gdt);
  g.d_k_bshk = Tensor::empty(k_bshk.dims(), gdt);
  g.d_v_bshv = Tensor::empty(v_bshv.dims(), gdt);
  g.d_erase_bshK = Tensor::empty(erase_bshK.dims(), DType::F32);
  g.d_write_bshV = Tensor::empty(write_bshV.dims(), DType::F32);
  if (g_bshK) g.d_g_bshK = Tensor::empty(g_bshK->dims(), DType::F32);
  g.d_state_bhkv = Tensor::empty(state_bhkv.dims(), DType::F32);
  dn_chunk_bwd_args a{};
  a.batch = d.batch;
  a.sequence = d.sequence;
  a.nheads = d.nheads;
  a.head_k_dim = d.head_k_dim;
  a.head_v_dim = d.head_v_dim;
  a.erase_width = erase_bshK.dim(3);
  a.write_width = write_bshV.dim(3);
  a.decay_width = g_bshK ? g_bshK->dim(3) : 0;
  a.has_gate = g_bshK ? 1 : 0;
  a.chunk_len = int32_t(chunk_len);
  a.scale = scale;
  a.qkv_dtype = int32_t(q_bshk.dtype());
  a.grad_dtype = int32_t(gdt);
  a.algo = DN_ALGO_AUTO;
  a.check_finite = check_finite ? 1 : 0;
  a.d_y = d_y_bshv.data();
  a.d_state_final =
      d_final_state_bhkv ? static_cast<const float*>(d_final_state_bhkv->data()) : nullptr;
  a.q = q_bshk.data();
  a.k = k_bshk.data();
  a.v = v_bshv.data();
  a.erase = static_cast<const float*>(erase_bshK.data());
  a.write = static_cast<const float*>(write_bshV.data());
  a.g = g_bshK ? static_cast<const float*>(g_bshK->data()) : nullptr;
  a.state_in = static_cast<const float*>(state_bhkv.data());
  a.d_q = g.d_q_bshk.data();
  a.d_k = g.d_k_bshk.data();
  a.d_v = g.d_v_bshv.data();
  a.d_erase = static_cast<float*>(g.d_erase_bshK.data());
  a.d_write = static_cast<float*>(g.d_write_bshV.data());
  a.d_g = g.d_g_bshK ? static_cast<float*>(g.d_g_bshK->data()) : nullptr;
  a.d_state = static_cast<float*>(g.d_state_bhkv.data());
  const size_t need = dn_chunk_bwd_workspace_bytes(&a);
  if (need) {
    a.workspace = (ws ? *ws : thread_workspace()).reserve(need, stream);
    a.workspace_bytes = need;
  }
  check(dn_chunk_bwd(&a, stream));
  return g;
}

// ---------------------------------------------------------------------------
// The projection front-end (qkv.rs:373-516) over dn_frontend.
// ---------------------------------------------------------------------------

Tensor ShortConv::zero_window(int64_t batch, DType dtype, hipStream_t stream) const {
  Tensor w = Tensor::empty({batch, conv_dim(), conv_kernel()}, dtype);
  check_hip(hipMemsetAsync(w.data(), 0, w.bytes(), stream), "hipMemsetAsync");
  return w;
}

int64_t QkvProjection::conv_dim() const {
  return key_dim() + n_householder * (key_dim() + value_dim());
}

int64_t QkvProjection::write_gate_width() const {
  switch (write_gate) {
    case WriteGate::Fixed: return 0;
    case WriteGate::Scalar: return n_householder * nheads;
    default: return n_householder * (key_dim() + value_dim());
  }
}

int64_t QkvProjection::d_in_proj() const {
  return conv_dim() + write_gate_width() + (has_gate ? value_dim() : 0) + extra_channels;
}

std::optional<Tensor> QkvProjection::zero_conv_window(int64_t batch, DType dtype,
                                                      hipStream_t stream) const {
  if (!conv) return std::nullopt;
  return conv->zero_window(batch, dtype, stream);
}

namespace {

struct FrontOut {
  Tensor q, k, v, erase, write;
  std::optional<Tensor> window;
};

FrontOut run_frontend(const QkvProjection& pr, const Tensor& projected, int64_t batch,
                      int64_t sequence, const std::optional<Tensor>& window,
                      std::optional<DType> out_dtype, hipStream_t stream) {
  require_defined(projected, "projection");
  if (projected.dim(projected.rank() - 1) != pr.d_in_proj())
    throw Error(DN_ERR_SHAPE, "projection: last axis must be d_in_proj = " +
                                  std::to_string(pr.d_in_proj()) + ", got " +
                                  std::to_string(projected.dim(projected.rank() - 1)));
  if (pr.conv.has_value() != window.has_value())  // qkv.rs:397-401
    throw Error(DN_ERR_SHAPE, "convolution window presence must match the block's convolution");
  const int64_t H = pr.nheads, dk = pr.head_k_dim, dv = pr.head_v_dim, u = pr.n_householder;
  const DType od = out_dtype.value_or(projected.dtype());
  FrontOut o;
  o.q = Tensor::empty({batch, sequence, H, dk}, od);
  o.k = Tensor::empty({batch, sequence * u, H, dk}, od);
  o.v = Tensor::empty({batch, sequence * u, H, dv}, od);
  if (pr.write_gate == WriteGate::Channel) {
    o.erase = Tensor::empty({batch, sequence * u, H, dk}, DType::F32);
    o.write = Tensor::empty({batch, sequence * u, H, dv}, DType::F32);
  } else {
    // One tensor for both halves, as the reference's (beta.clone(), beta).
    o.erase = Tensor::empty({batch, sequence * u, H, 1}, DType::F32);
    o.write = o.erase;
  }
  dn_frontend_args a{};
  a.batch = batch;
  a.sequence = sequence;
  a.nheads = H;
  a.head_k_dim = dk;
  a.head_v_dim = dv;
  a.n_householder = u;
  a.conv_kernel = pr.conv_kernel();
  a.proj_stride = pr.d_in_proj();
  a.conv_activation = pr.conv ? int32_t(pr.conv->activation) : DN_ACT_IDENTITY;
  a.qk_activation = int32_t(pr.qk_activation);
  a.qk_norm = int32_t(pr.qk_norm);
  a.write_gate = int32_t(pr.write_gate);
  a.allow_neg_eigval = pr.allow_neg_eigval ? 1 : 0;
  a.in_dtype = int32_t(projected.dtype());
  a.out_dtype = int32_t(od);
  a.projected = projected.data();
  if (pr.conv) {
    require_f32(pr.conv->weight, "conv weight");
    expect_shape(*window, {batch, pr.conv_dim(), pr.conv_kernel()}, "conv window");
    if (window->dtype() != projected.dtype())
      throw Error(DN_ERR_DTYPE, "conv window: dtype must be the projection's");
    a.conv_weight = static_cast<const float*>(pr.conv->weight.data());
    if (pr.conv->bias) {
      require_f32(*pr.conv->bias, "conv bias");
      a.conv_bias = static_cast<const float*>(pr.conv->bias->data());
    }
    o.window = Tensor::empty(window->dims(), window->dtype());
    a.window_in = window->data();
    a.window_out = o.window->data();
  }
  a.q = o.q.data();
  a.k = o.k.data();
  a.v = o.v.data();
  a.erase = static_cast<float*>(o.erase.data());
  a.write = static_cast<float*>(o.write.data());
  check(dn_frontend(&a, stream));
  return o;
}

}  // namespace

std::pair<Qkv, std::optional<Tensor>> QkvProjection::forward_projected(
    const Tensor& projected_bsw, const std::optional<Tensor>& conv_window_bwc,
    hipStream_t stream, std::optional<DType> out_dtype) const {
  if (projected_bsw.rank() != 3)
    throw Error(DN_ERR_SHAPE, "projection: expected [batch, sequence, d_in_proj]");
  FrontOut o = run_frontend(*this, projected_bsw, projected_bsw.dim(0), projected_bsw.dim(1),
                            conv_window_bwc, out_dtype, stream);
  return {Qkv{o.q, o.k, o.v, o.erase, o.write}, o.window};
}

std::pair<QkvStep, std::optional<Tensor>> QkvProjection::step_projected(
    const Tensor& projected_bw, const std::optional<Tensor>& conv_window_bwc,
    hipStream_t stream, std::optional<DType> out_dtype) const {
  if (projected_bw.rank() != 2)
    throw Error(DN_ERR_SHAPE, "projection: expected [batch, d_in_proj]");
  const int64_t B = projected_bw.dim(0);
  FrontOut o = run_frontend(*this, projected_bw, B, 1, conv_window_bwc, out_dtype, stream);
  return {QkvStep{o.q.reshape({B, nheads, head_k_dim}), o.k, o.v, o.erase, o.write}, o.window};
}

Tensor OutNorm::forward(const Tensor& x, const std::optional<Tensor>& gate,
                       int64_t gate_token_stride, hipStream_t stream,
                       std::optional<DType> out_dtype) const {
  // norm.rs:131-132
  if (gated && !gate) throw Error(DN_ERR_NULL, "OutNorm::Gated needs an output gate");
  if (!gated && gate) throw Error(DN_ERR_SHAPE, "OutNorm::Plain takes no output gate");
  require_defined(x, "x");
  require_f32(weight, "norm weight");
  if (x.rank() < 2) throw Error(DN_ERR_SHAPE, "x: expected [.., nheads, head_v_dim]");
  const int64_t H = x.dim(x.rank() - 2), D = x.dim(x.rank() - 1);
  if (weight.numel() != size_t(D))
    throw Error(DN_ERR_SHAPE, "norm weight: expected " + std::to_string(D) + " values");
  Tensor out = Tensor::empty(x.dims(), out_dtype.value_or(x.dtype()));
  dn_out_norm_args a{};
  a.tokens = int64_t(x.numel()) / (H * D);
  a.nheads = H;
  a.head_v_dim = D;
  a.gate_stride = gate ? (gate_token_stride ? gate_token_stride : H * D) : 0;
  a.eps = eps;
  a.x_dtype = int32_t(x.dtype());
  a.gate_dtype = gate ? int32_t(gate->dtype()) : DN_F32;
  a.out_dtype = int32_t(out.dtype());
  a.x = x.data();
  a.gate = gate ? gate->data() : nullptr;
  a.weight = static_cast<const float*>(weight.data());
  a.out = out.data();
  check(dn_out_norm(&a, stream));
  return out;
}

Tensor block_step(const QkvProjection& proj, const OutNorm& norm, const Tensor& projected_bw,
                  const std::optional<Tensor>& conv_window_bwc,
                  const std::optional<Tensor>& g_bhK, Tensor& state_bhkv, double scale,
                  hipStream_t stream, std::optional<DType> out_dtype, bool check_finite) {
  require_defined(projected_bw, "projected");
  if (projected_bw.rank() != 2 || projected_bw.dim(1) != proj.d_in_proj())
    throw Error(DN_ERR_SHAPE, "projected: expected [batch, " + std::to_string(proj.d_in_proj()) +
                                  "]");
  if (proj.n_householder != 1)
    throw Error(DN_ERR_UNSUPPORTED, "dn_block_step serves n_householder = 1");
  if (proj.conv.has_value() != conv_window_bwc.has_value())
    throw Error(DN_ERR_SHAPE, "convolution window presence must match the block's convolution");
  if (norm.gated && !proj.has_gate)
    throw Error(DN_ERR_NULL, "OutNorm::Gated needs the projection's output gate");
  if (proj.has_gate && !norm.gated)
    throw Error(DN_ERR_SHAPE, "OutNorm::Plain takes no output gate");  // norm.rs OutNorm::forward
  const int64_t B = projected_bw.dim(0), H = proj.nheads, dk = proj.head_k_dim,
                dv = proj.head_v_dim;
  require_f32(state_bhkv, "state");
  if (state_bhkv.dims() != std::vector<int64_t>{B, H, dk, dv})
    throw Error(DN_ERR_SHAPE, "state: expected [batch, nheads, head_k_dim, head_v_dim]");
  if (g_bhK) require_f32(*g_bhK, "forget gate");
  require_f32(norm.weight, "norm weight");
  if (conv_window_bwc && conv_window_bwc->dtype() != projected_bw.dtype())
    throw Error(DN_ERR_DTYPE, "conv window: expected the projection's dtype");
  Tensor out = Tensor::empty({B, H, dv}, out_dtype.value_or(projected_bw.dtype()));
  dn_block_step_args a{};
  a.batch = B;
  a.nheads = H;
  a.head_k_dim = dk;
  a.head_v_dim = dv;
  a.conv_kernel = proj.conv_kernel();
  a.proj_stride = proj.d_in_proj();
  a.conv_activation = proj.conv ? int32_t(proj.conv->activation) : DN_ACT_IDENTITY;
  a.qk_activation = int32_t(proj.qk_activation);
  a.qk_norm = int32_t(proj.qk_norm);
  a.write_gate = int32_t(proj.write_gate);
  a.allow_neg_eigval = proj.allow_neg_eigval;
  a.in_dtype = int32_t(projected_bw.dtype());
  a.out_dtype = int32_t(out.dtype());
  a.has_gate = g_bhK.has_value();
  a.decay_width = g_bhK ? g_bhK->dim(g_bhK->rank() - 1) : 0;
  a.scale = scale;
  a.eps = norm.eps;
  a.norm_gated = norm.gated;
  a.check_finite = check_finite;
  a.projected = projected_bw.data();
  if (proj.conv) {
    require_f32(proj.conv->weight, "conv weight");
    a.conv_weight = static_cast<const float*>(proj.conv->weight.data());
    a.conv_bias = proj.conv->bias ? static_cast<const float*>(proj.conv->bias->data()) : nullptr;
    a.window_in = conv_window_bwc->data();
    a.window_out = conv_window_bwc->data();
  }
  a.g = g_bhK ? static_cast<const float*>(g_bhK->data()) : nullptr;
  a.state_in = static_cast<const float*>(state_bhkv.data());
  a.state_out = static_cast<float*>(state_bhkv.data());
  a.norm_weight = static_cast<const float*>(norm.weight.data());
  a.out = out.data();
  check(dn_block_step(&a, stream));
  return out;
}

}  // namespace deltanet
