// deltanet.hpp — C++ host interface of the MI355X delta-rule core.
//
// Mirrors the Rust interface of burn-deltanet's delta-rule core with the same
// names, argument meaning and error behaviour, over device tensors:
//   DeltaPath, DeltaInput::{dims, resolved_scale, has_channel_decay, sanity,
//   run, delta_recurrent, delta_chunk_recalculated}, beta_gates
//                                         src/delta/path.rs:21-231
//   delta_step                            src/delta/recurrent.rs:41-99
//   DeltaChunkGrads, combined_backward    src/delta/chunk_recalculated/
//                                         combined_backward.rs:50-189
//   TriSolve, unit_lower_inverse          src/delta/tri.rs:53-114
//   QkvProjection, OutNorm, block_step    src/common/qkv.rs, norm.rs, and
//                                         gated_deltanet_1.rs:218-234
// Every computation is a call through the C ABI of deltanet_core.h. Where
// the reference panics on an assert!, these functions throw deltanet::Error
// carrying the same message (and the dn_status the C ABI uses for it).
//
// The reference is functional: its functions return fresh tensors, and so do
// these (device memory owned by the returned Tensor). delta_step_in_place is
// the one addition: the in-place state update a decode loop wants.
//
// Library: libdeltanet.so (links libdeltanet_core.so and libamdhip64.so).
#ifndef DELTANET_HPP
#define DELTANET_HPP

#include <cstddef>
#include <cstdint>
#include <memory>
#include <optional>
#include <stdexcept>
#include <string>
#include <utility>
#include <vector>

#include "deltanet_core.h"

namespace deltanet {

enum class DType : int32_t { F32 = DN_F32, BF16 = DN_BF16 };

size_t dtype_size(DType dtype);

// The reference's assert! failures, as exceptions. status() is the dn_status
// the C ABI returns for the same condition.
class Error : public std::runtime_error {
 public:
  Error(int status, const std::string& what);
  int status() const noexcept { return status_; }

 private:
  int status_;
};

// A dense row-major device tensor: either owning (reference-counted device
// memory from Tensor::empty) or a view of memory the caller owns.
class Tensor {
 public:
  Tensor() = default;
  // Fresh device allocation (contents undefined).
  static Tensor empty(std::vector<int64_t> dims, DType dtype);
  // Non-owning view of `data` (device memory the caller keeps alive).
  static Tensor view(void* data, std::vector<int64_t> dims, DType dtype);

  bool defined() const { return data_ != nullptr; }
  int rank() const { return int(dims_.size()); }
  int64_t dim(int axis) const { return dims_.at(size_t(axis)); }
  const std::vector<int64_t>& dims() const { return dims_; }
  DType dtype() const { return dtype_; }
  void* data() const { return data_; }
  size_t numel() const;
  size_t bytes() const { return numel() * dtype_size(dtype_); }
  // Same storage, new shape of the same element count.
  Tensor reshape(std::vector<int64_t> dims) const;

 private:
  std::shared_ptr<void> owner_;
  void* data_ = nullptr;
  std::vector<int64_t> dims_;
  DType dtype_ = DType::F32;
};

// Device scratch for the chunk calls (dn_chunk_fwd / dn_chunk_bwd), owned by
// the caller of this mirror, so no call falls back on the library's shared
// pool. reserve() grows it on the stream it is used on: the old buffer is
// released and the new one taken stream-ordered (hipFreeAsync /
// hipMallocAsync), so growth neither drains the device nor frees memory a
// queued call still reads. A Workspace serves one stream at a time; calls
// on two streams at once need one each. The functions below that take a
// `Workspace*` use the calling thread's own per-device Workspace when it is
// null.
class Workspace {
 public:
  Workspace() = default;
  ~Workspace();
  Workspace(const Workspace&) = delete;
  Workspace& operator=(const Workspace&) = delete;
  // At least `bytes` of device memory for work queued on `stream`.
  void* reserve(size_t bytes, hipStream_t stream);
  size_t capacity() const { return bytes_; }

 private:
  void* ptr_ = nullptr;
  size_t bytes_ = 0;
};

// How the WY transform's (I − N)⁻¹ is evaluated (src/delta/tri.rs:53-64).
// Inside the chunk paths both evaluate the same exact inverse (the
// reference's Neumann series is a test baseline there); unit_lower_inverse
// honours the variant.
enum class TriSolve { Blocked, Neumann };

// tri.rs:66-114: T = (I − N)⁻¹ for a batched strictly lower triangular N of
// shape [..., size, size], float32. Blocked reads only N's strict lower
// triangle; Neumann sums I + N + … + N^{size−1} term by term over the whole
// matrix, up to DN_TRI_NEUMANN_MAX_SIZE. The caller owes the strict lower
// property, as in the reference.
Tensor unit_lower_inverse(const Tensor& n_strict, TriSolve solve = TriSolve::Blocked,
                          hipStream_t stream = nullptr, bool check_finite = false);

// Which evaluation of the delta rule runs (src/delta/path.rs:21-99).
struct DeltaPath {
  enum class Kind { Recurrent, Chunk, ChunkRecalculated };
  static constexpr int64_t DEFAULT_CHUNK_LEN = 64;

  Kind kind = Kind::ChunkRecalculated;
  std::optional<int64_t> chunk_len;  // nullopt ⇒ DEFAULT_CHUNK_LEN
  TriSolve solve = TriSolve::Blocked;

  static DeltaPath recurrent() { return DeltaPath{Kind::Recurrent, std::nullopt, TriSolve::Blocked}; }
  // The default: chunkwise at the default chunk length and backward.
  static DeltaPath chunk() { return DeltaPath{}; }
  // DeltaPath::chunk_len(n) of the reference (a static and a field cannot
  // share a name in C++).
  static DeltaPath with_chunk_len(int64_t n) {
    return DeltaPath{Kind::ChunkRecalculated, n, TriSolve::Blocked};
  }
  static DeltaPath chunk_len_on_tape(int64_t n) { return DeltaPath{Kind::Chunk, n, TriSolve::Blocked}; }
  // Recurrent answers 1: it is the chunk length of a token-at-a-time pass.
  int64_t resolved_chunk_len() const {
    return kind == Kind::Recurrent ? 1 : chunk_len.value_or(DEFAULT_CHUNK_LEN);
  }
};

// (erase, write) for a per-head β: the same values broadcast over both
// channel axes. [batch, .., nheads] → two views [batch, .., nheads, 1].
std::pair<Tensor, Tensor> beta_gates(const Tensor& beta);

// Everything the delta-rule core consumes (src/delta/path.rs:120-141).
// q/k arrive L2-normalised and unscaled; gates arrive squashed (g = log α ≤ 0).
// q, k, v share one dtype (f32 or bf16); gates and state are f32.
struct DeltaInput {
  Tensor q_bshk;       // [batch, sequence, nheads, head_k_dim]
  Tensor k_bshk;       // [batch, sequence, nheads, head_k_dim]
  Tensor v_bshv;       // [batch, sequence, nheads, head_v_dim]
  Tensor erase_bshK;   // [batch, sequence, nheads, 1 | head_k_dim]
  Tensor write_bshV;   // [batch, sequence, nheads, 1 | head_v_dim]
  std::optional<Tensor> g_bshK;  // [batch, sequence, nheads, 1 | head_k_dim]
  Tensor state_bhkv;   // [batch, nheads, head_k_dim, head_v_dim]
  std::optional<double> scale;   // nullopt ⇒ 1/√head_k_dim

  struct Dims {
    int64_t batch, sequence, nheads, head_k_dim, head_v_dim;
  };
  Dims dims() const;
  double resolved_scale() const;
  bool has_channel_decay() const;
  // Shape and gate-width checks (path.rs:177-197). The NaN/Inf guards of
  // the reference's check-nan/check-inf features run on the device when a
  // call is made with check_finite = true.
  void sanity() const;
  // path.rs:215-231. Returns (y_bshv, final_state_bhkv).
  std::pair<Tensor, Tensor> run(const DeltaPath& path = DeltaPath{}, hipStream_t stream = nullptr,
                                bool check_finite = false, Workspace* ws = nullptr) const;
  // recurrent.rs:107-142: delta_step unrolled over the sequence.
  std::pair<Tensor, Tensor> delta_recurrent(hipStream_t stream = nullptr,
                                            bool check_finite = false) const;
  // chunk_recalculated.rs:36-83 → DeltaChunkBackendExt::delta_chunk_recalculated.
  std::pair<Tensor, Tensor> delta_chunk_recalculated(int64_t chunk_len,
                                                     hipStream_t stream = nullptr,
                                                     bool check_finite = false,
                                                     Workspace* ws = nullptr) const;
};

// recurrent.rs:41-99. Returns (y_bhv, next_state_bhkv).
std::pair<Tensor, Tensor> delta_step(const Tensor& q_bhk, const Tensor& k_bhk, const Tensor& v_bhv,
                                     const Tensor& erase_bhK, const Tensor& write_bhV,
                                     const std::optional<Tensor>& g_bhK, const Tensor& state_bhkv,
                                     double scale, hipStream_t stream = nullptr,
                                     bool check_finite = false);

// delta_step with the state updated in place and y written to `y_bhv`.
void delta_step_in_place(const Tensor& q_bhk, const Tensor& k_bhk, const Tensor& v_bhv,
                         const Tensor& erase_bhK, const Tensor& write_bhV,
                         const std::optional<Tensor>& g_bhK, Tensor& state_bhkv, Tensor& y_bhv,
                         double scale, hipStream_t stream = nullptr, bool check_finite = false);

// combined_backward.rs:50-65: gradients of the seven leaves. d_erase,
// d_write and d_g have their gate's own width; d_g is with respect to g.
struct DeltaChunkGrads {
  Tensor d_q_bshk, d_k_bshk, d_v_bshv, d_erase_bshK, d_write_bshV;
  std::optional<Tensor> d_g_bshK;
  Tensor d_state_bhkv;
};

// combined_backward.rs:72-189. d_final_state_bhkv = nullopt means zeros.
DeltaChunkGrads combined_backward(const Tensor& d_y_bshv,
                                  const std::optional<Tensor>& d_final_state_bhkv,
                                  const Tensor& q_bshk, const Tensor& k_bshk, const Tensor& v_bshv,
                                  const Tensor& erase_bshK, const Tensor& write_bshV,
                                  const std::optional<Tensor>& g_bshK, const Tensor& state_bhkv,
                                  int64_t chunk_len, double scale, hipStream_t stream = nullptr,
                                  bool check_finite = false, Workspace* ws = nullptr);

// ---------------------------------------------------------------------------
// The projection front-end (src/common/qkv.rs, conv.rs, norm.rs) over
// dn_frontend: everything QkvProjection does after its in_proj GEMM, which
// stays with the caller (the reference's Burn Linear). n_value_heads =
// nheads; QkNorm::Sum is refused (both depend on burn_stack code the
// reference does not vendor).
// ---------------------------------------------------------------------------

enum class QkActivation : int32_t {  // norm.rs:22-34
  Identity = DN_ACT_IDENTITY,
  Silu = DN_ACT_SILU,
  Relu = DN_ACT_RELU,
  EluPlusOne = DN_ACT_ELU_PLUS_ONE
};
enum class ConvActivation : int32_t { Silu = DN_ACT_SILU, Identity = DN_ACT_IDENTITY };  // conv.rs:29-35
enum class QkNorm : int32_t { L2 = DN_QKNORM_L2, Sum = DN_QKNORM_SUM, None = DN_QKNORM_NONE };
enum class WriteGate : int32_t {  // qkv.rs:45-54
  Fixed = DN_WRITE_FIXED,
  Scalar = DN_WRITE_SCALAR,
  Channel = DN_WRITE_CHANNEL
};

// conv.rs:49-83: the depthwise weight [conv_dim, conv_kernel] (Conv1d's
// [conv_dim, 1, kernel] without its unit axis), float32.
struct ShortConv {
  Tensor weight;
  std::optional<Tensor> bias;  // [conv_dim], float32
  ConvActivation activation = ConvActivation::Silu;

  int64_t conv_dim() const { return weight.dim(0); }
  int64_t conv_kernel() const { return weight.dim(weight.rank() - 1); }
  // A zero rolling window [batch, conv_dim, conv_kernel] ("no previous tokens").
  Tensor zero_window(int64_t batch, DType dtype, hipStream_t stream = nullptr) const;
};

// qkv.rs:76-97. The output gate and the extra channels are column ranges of
// the projection (qkv.rs:267-300), left to the caller.
struct Qkv {
  Tensor q_bshk, k_bShk, v_bShv, erase_bShK, write_bShV;
};
// qkv.rs:99-116.
struct QkvStep {
  Tensor q_bhk, k_buhk, v_buhv, erase_buhK, write_buhV;
};

// qkv.rs:118-155.
struct QkvProjection {
  int64_t nheads = 1, head_k_dim = 1, head_v_dim = 1, n_householder = 1;
  std::optional<ShortConv> conv;
  QkActivation qk_activation = QkActivation::Silu;
  QkNorm qk_norm = QkNorm::L2;
  WriteGate write_gate = WriteGate::Scalar;
  bool has_gate = false;
  bool allow_neg_eigval = false;
  int64_t extra_channels = 0;

  int64_t key_dim() const { return nheads * head_k_dim; }
  int64_t value_dim() const { return nheads * head_v_dim; }
  int64_t conv_dim() const;          // qkv.rs:180-182
  int64_t write_gate_width() const;  // qkv.rs:189-197
  int64_t d_in_proj() const;         // qkv.rs:199-205
  int64_t conv_kernel() const { return conv ? conv->conv_kernel() : 0; }
  std::optional<Tensor> zero_conv_window(int64_t batch, DType dtype,
                                         hipStream_t stream = nullptr) const;

  // QkvProjection::forward after in_proj (qkv.rs:373-449): projected
  // [batch, sequence, d_in_proj] → the delta rule's inputs and the next
  // window. q, k, v take `out_dtype` (default: the projection's dtype).
  std::pair<Qkv, std::optional<Tensor>> forward_projected(
      const Tensor& projected_bsw, const std::optional<Tensor>& conv_window_bwc,
      hipStream_t stream = nullptr, std::optional<DType> out_dtype = std::nullopt) const;
  // QkvProjection::step after in_proj (qkv.rs:454-516): projected
  // [batch, d_in_proj].
  std::pair<QkvStep, std::optional<Tensor>> step_projected(
      const Tensor& projected_bw, const std::optional<Tensor>& conv_window_bwc,
      hipStream_t stream = nullptr, std::optional<DType> out_dtype = std::nullopt) const;
};

// OutNorm (src/common/norm.rs:106-144): RMSNorm over head_v_dim per head,
// weight gamma [head_v_dim] (float32); gated, times silu(gate) after the norm.
// eps is burn_stack's RmsNorm epsilon, which the reference does not vendor
// (1e-5, Burn's RmsNorm default, unless set).
struct OutNorm {
  Tensor weight;
  bool gated = true;
  double eps = 1e-5;

  // x [.., nheads, head_v_dim]. The gate, when gated, is nheads·head_v_dim
  // values per token starting at gate.data(), tokens gate_token_stride
  // elements apart (0: packed, as x) — a column range of the projection
  // (qkv.rs:429) is passed as a view of its first element and d_in_proj.
  Tensor forward(const Tensor& x, const std::optional<Tensor>& gate = std::nullopt,
                 int64_t gate_token_stride = 0, hipStream_t stream = nullptr,
                 std::optional<DType> out_dtype = std::nullopt) const;
};

// One decode token of a delta-rule block between in_proj and out_proj in one
// launch (dn_block_step): proj.step_projected, delta_step and norm.forward as
// gated_deltanet_1.rs:218-234 runs them, given the forget gate g = log α
// [batch, nheads, 1 | head_k_dim] (nullopt: no decay); q, k, v and y stay in
// fp32 between the stages. The state [batch, nheads, head_k_dim, head_v_dim]
// and the conv window are updated in place; returns out [batch, nheads,
// head_v_dim] in `out_dtype` (default: the projection's dtype).
// n_householder = 1, head dims up to DN_BLOCK_STEP_MAX_HEAD_DIM.
Tensor block_step(const QkvProjection& proj, const OutNorm& norm, const Tensor& projected_bw,
                  const std::optional<Tensor>& conv_window_bwc,
                  const std::optional<Tensor>& g_bhK, Tensor& state_bhkv, double scale,
                  hipStream_t stream = nullptr, std::optional<DType> out_dtype = std::nullopt,
                  bool check_finite = false);

}  // namespace deltanet

#endif  // DELTANET_HPP
