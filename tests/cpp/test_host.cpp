// Tests of the C++ host mirror (include/deltanet.hpp), in the manner of the
// reference's own tests of src/delta (src/delta/tests.rs): shape/gate-width
// assertions, the algorithm selector, and the forward / step / backward
// values against the CPU oracle (oracle/liboracle.so, float64).
//
//   test_host --host-only   argument checks only; no HIP call is made
//   test_host --gpu         everything (needs a GPU)
//
// Prints "ok <case>" per case; exits nonzero at the first failure.

#include <hip/hip_runtime_api.h>

#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <functional>
#include <string>
#include <vector>

#include "deltanet.hpp"

extern "C" {
int or_chunk_fwd_f64(long B, long S, long H, long K, long V, long ew, long ww, long dw, long L,
                     const double* q, const double* k, const double* v, const double* erase,
                     const double* write, const double* g, const double* state, double scale,
                     double* y, double* state_out);
int or_delta_step_f64(long B, long H, long K, long V, long ew, long ww, long dw, const double* q,
                      const double* k, const double* v, const double* erase, const double* write,
                      const double* g, const double* state, double scale, double* y,
                      double* state_out);
int or_chunk_bwd_f64(long B, long S, long H, long K, long V, long ew, long ww, long dw, long L,
                     const double* dy, const double* dstate, const double* q, const double* k,
                     const double* v, const double* erase, const double* write, const double* g,
                     const double* state, double scale, double* dq, double* dk, double* dv,
                     double* de, double* dwr, double* dg, double* dstate_out);
}

using namespace deltanet;
using Vec = std::vector<double>;

namespace {

[[noreturn]] void fail(const std::string& what) {
  std::fprintf(stderr, "FAIL %s\n", what.c_str());
  std::fflush(stderr);
  std::exit(1);
}

void ok(const char* name) {
  std::printf("ok %s\n", name);
  std::fflush(stdout);
}

// Expect `fn` to throw deltanet::Error with this status and message.
void expect_error(const char* name, int status, const std::string& message,
                  const std::function<void()>& fn) {
  try {
    fn();
  } catch (const Error& e) {
    if (e.status() != status || message != e.what())
      fail(std::string(name) + ": got status " + std::to_string(e.status()) + " \"" + e.what() +
           "\"; want " + std::to_string(status) + " \"" + message + "\"");
    ok(name);
    return;
  }
  fail(std::string(name) + ": no error raised");
}

// splitmix64 + Box–Muller.
struct Rng {
  uint64_t s;
  explicit Rng(uint64_t seed) : s(seed) {}
  uint64_t next() {
    uint64_t z = (s += 0x9e3779b97f4a7c15ull);
    z = (z ^ (z >> 30)) * 0xbf58476d1ce4e5b9ull;
    z = (z ^ (z >> 27)) * 0x94d049bb133111ebull;
    return z ^ (z >> 31);
  }
  double uniform() { return (double(next() >> 11) + 0.5) * (1.0 / 9007199254740992.0); }
  double normal() {
    const double u1 = uniform(), u2 = uniform();
    return std::sqrt(-2.0 * std::log(u1)) * std::cos(6.283185307179586 * u2);
  }
  Vec normals(size_t n, double std_ = 1.0) {
    Vec x(n);
    for (auto& v : x) v = std_ * normal();
    return x;
  }
};

Vec l2_rows(Vec x, size_t width) {
  for (size_t r = 0; r < x.size() / width; ++r) {
    double ss = 0;
    for (size_t c = 0; c < width; ++c) ss += x[r * width + c] * x[r * width + c];
    const double inv = 1.0 / std::sqrt(ss + 1e-6);
    for (size_t c = 0; c < width; ++c) x[r * width + c] *= inv;
  }
  return x;
}
Vec sigmoid(Vec x) {
  for (auto& v : x) v = 1.0 / (1.0 + std::exp(-v));
  return x;
}
Vec neg_softplus(Vec x, double s) {
  for (auto& v : x) v = -std::log1p(std::exp(v)) * s;
  return x;
}

uint16_t to_bf16(float f) {
  uint32_t u;
  std::memcpy(&u, &f, 4);
  u += 0x7fffu + ((u >> 16) & 1u);
  return uint16_t(u >> 16);
}
float from_bf16(uint16_t h) {
  const uint32_t u = uint32_t(h) << 16;
  float f;
  std::memcpy(&f, &u, 4);
  return f;
}

void hip_ok(hipError_t e, const char* what) {
  if (e != hipSuccess) fail(std::string(what) + ": " + hipGetErrorString(e));
}

// Upload as `dtype`; `x` is replaced by the values the device holds (bf16
// rounding), so the oracle sees exactly what the GPU reads.
Tensor upload(Vec& x, std::vector<int64_t> dims, DType dtype) {
  Tensor t = Tensor::empty(std::move(dims), dtype);
  if (t.numel() != x.size()) fail("upload: size mismatch");
  if (dtype == DType::F32) {
    std::vector<float> h(x.begin(), x.end());
    for (size_t i = 0; i < x.size(); ++i) x[i] = h[i];
    hip_ok(hipMemcpy(t.data(), h.data(), t.bytes(), hipMemcpyHostToDevice), "hipMemcpy");
  } else {
    std::vector<uint16_t> h(x.size());
    for (size_t i = 0; i < x.size(); ++i) {
      h[i] = to_bf16(float(x[i]));
      x[i] = from_bf16(h[i]);
    }
    hip_ok(hipMemcpy(t.data(), h.data(), t.bytes(), hipMemcpyHostToDevice), "hipMemcpy");
  }
  return t;
}

Vec download(const Tensor& t) {
  hip_ok(hipDeviceSynchronize(), "hipDeviceSynchronize");
  Vec x(t.numel());
  if (t.dtype() == DType::F32) {
    std::vector<float> h(t.numel());
    hip_ok(hipMemcpy(h.data(), t.data(), t.bytes(), hipMemcpyDeviceToHost), "hipMemcpy");
    for (size_t i = 0; i < x.size(); ++i) x[i] = h[i];
  } else {
    std::vector<uint16_t> h(t.numel());
    hip_ok(hipMemcpy(h.data(), t.data(), t.bytes(), hipMemcpyDeviceToHost), "hipMemcpy");
    for (size_t i = 0; i < x.size(); ++i) x[i] = from_bf16(h[i]);
  }
  return x;
}

// Normwise relative error max|a − b| / max|b|.
double rel_err(const Vec& a, const Vec& b) {
  double num = 0, den = 0;
  for (size_t i = 0; i < a.size(); ++i) {
    num = std::max(num, std::fabs(a[i] - b[i]));
    den = std::max(den, std::fabs(b[i]));
  }
  return num / (den > 0 ? den : 1.0);
}

void expect_close(const char* name, const Vec& got, const Vec& want, double tol) {
  if (got.size() != want.size()) fail(std::string(name) + ": size mismatch");
  for (double x : got)
    if (!std::isfinite(x)) fail(std::string(name) + ": non-finite value");
  const double e = rel_err(got, want);
  if (!(e <= tol)) fail(std::string(name) + ": relative error " + std::to_string(e));
}

// ---------------------------------------------------------------------------
// Argument checks (no device memory is touched: views of a dummy address).
// ---------------------------------------------------------------------------
void host_cases() {
  void* fake = reinterpret_cast<void*>(uintptr_t(0x1000));
  auto v4 = [&](std::vector<int64_t> d, DType t = DType::F32) { return Tensor::view(fake, d, t); };
  const int64_t B = 2, S = 9, H = 2, K = 4, V = 6;
  auto good = [&]() {
    return DeltaInput{v4({B, S, H, K}), v4({B, S, H, K}), v4({B, S, H, V}), v4({B, S, H, 1}),
                      v4({B, S, H, 1}), v4({B, S, H, 1}), v4({B, H, K, V}), std::nullopt};
  };
  good().sanity();
  ok("sanity_accepts_broadcast_gates");
  {
    DeltaInput in = good();
    in.erase_bshK = v4({B, S, H, K});
    in.write_bshV = v4({B, S, H, V});
    in.g_bshK = v4({B, S, H, K});
    in.sanity();
    if (!in.has_channel_decay()) fail("has_channel_decay: per-channel g not seen");
    if (good().has_channel_decay()) fail("has_channel_decay: per-head g seen as per-channel");
    ok("sanity_accepts_channel_gates");
  }
  expect_error("k_shape", DN_ERR_SHAPE, "k: expected shape [2, 9, 2, 4], got [2, 9, 2, 5]", [&] {
    DeltaInput in = good();
    in.k_bshk = v4({B, S, H, 5});
    in.sanity();
  });
  expect_error("state_shape", DN_ERR_SHAPE, "state: expected shape [2, 2, 4, 6], got [2, 2, 6, 4]",
               [&] {
                 DeltaInput in = good();
                 in.state_bhkv = v4({B, H, V, K});
                 in.sanity();
               });
  expect_error("erase_width", DN_ERR_GATE_WIDTH, "erase gate: last axis must be 1 or 4, got 3",
               [&] {
                 DeltaInput in = good();
                 in.erase_bshK = v4({B, S, H, 3});
                 in.sanity();
               });
  expect_error("write_width", DN_ERR_GATE_WIDTH, "write gate: last axis must be 1 or 6, got 4",
               [&] {
                 DeltaInput in = good();
                 in.write_bshV = v4({B, S, H, 4});
                 in.sanity();
               });
  expect_error("forget_width", DN_ERR_GATE_WIDTH, "forget gate: last axis must be 1 or 4, got 6",
               [&] {
                 DeltaInput in = good();
                 in.g_bshK = v4({B, S, H, 6});
                 in.sanity();
               });
  expect_error("gate_leading_dims", DN_ERR_SHAPE,
               "erase gate: expected leading dims [2, 9, 2], got [2, 8, 2, 1]", [&] {
                 DeltaInput in = good();
                 in.erase_bshK = v4({B, S - 1, H, 1});
                 in.sanity();
               });
  expect_error("empty_sequence", DN_ERR_SEQUENCE, "sequence length must be at least 1", [&] {
    DeltaInput in{v4({B, 0, H, K}), v4({B, 0, H, K}), v4({B, 0, H, V}), v4({B, 0, H, 1}),
                  v4({B, 0, H, 1}), std::nullopt, v4({B, H, K, V}), std::nullopt};
    in.run();
  });
  expect_error("chunk_len_zero", DN_ERR_CHUNK_LEN, "chunk_len must be at least 1",
               [&] { good().run(DeltaPath::with_chunk_len(0)); });
  {
    QkvProjection pr;
    pr.nheads = 2;
    pr.head_k_dim = 4;
    pr.head_v_dim = 6;
    pr.n_householder = 2;
    Tensor st = Tensor::view(fake, {1, 2, 4, 6}, DType::F32);
    expect_error("block_step_householder", DN_ERR_UNSUPPORTED,
                 "dn_block_step serves n_householder = 1", [&] {
                   block_step(pr, OutNorm{Tensor::view(fake, {6}, DType::F32), false},
                              Tensor::view(fake, {1, pr.d_in_proj()}, DType::F32), std::nullopt,
                              std::nullopt, st, 0.5);
                 });
  }
  // tri.rs:74-79.
  expect_error("tri_square_block", DN_ERR_SHAPE, "unit_lower_inverse expects a square trailing block",
               [&] { unit_lower_inverse(v4({3, 4, 5})); });
  expect_error("tri_dtype", DN_ERR_DTYPE, "unit_lower_inverse: n_strict must be float32",
               [&] { unit_lower_inverse(v4({3, 4, 4}, DType::BF16)); });
  expect_error("qkv_dtypes", DN_ERR_DTYPE, "q, k and v must share one dtype", [&] {
    DeltaInput in = good();
    in.q_bshk = v4({B, S, H, K}, DType::BF16);
    in.sanity();
  });
  expect_error("gate_dtype", DN_ERR_DTYPE, "erase gate: gates and state must be float32", [&] {
    DeltaInput in = good();
    in.erase_bshK = v4({B, S, H, 1}, DType::BF16);
    in.sanity();
  });
  expect_error("step_state_shape", DN_ERR_SHAPE,
               "state: expected shape [2, 2, 4, 6], got [2, 2, 4, 5]", [&] {
                 delta_step(v4({B, H, K}), v4({B, H, K}), v4({B, H, V}), v4({B, H, 1}),
                            v4({B, H, 1}), std::nullopt, v4({B, H, K, 5}), 0.5);
               });
  expect_error("step_erase_width", DN_ERR_GATE_WIDTH,
               "erase gate: last axis must be 1 or 4, got 2", [&] {
                 delta_step(v4({B, H, K}), v4({B, H, K}), v4({B, H, V}), v4({B, H, 2}),
                            v4({B, H, 1}), std::nullopt, v4({B, H, K, V}), 0.5);
               });
  expect_error("backward_dy_shape", DN_ERR_SHAPE, "d_y: expected shape [2, 9, 2, 6], got [2, 9, 2, 4]",
               [&] {
                 DeltaInput in = good();
                 combined_backward(v4({B, S, H, K}), std::nullopt, in.q_bshk, in.k_bshk, in.v_bshv,
                                   in.erase_bshK, in.write_bshV, in.g_bshK, in.state_bhkv, 16,
                                   0.5);
               });
  // The algorithm selector (path.rs:21-99).
  if (DeltaPath::recurrent().resolved_chunk_len() != 1 ||
      DeltaPath::chunk().resolved_chunk_len() != DeltaPath::DEFAULT_CHUNK_LEN ||
      DeltaPath{}.kind != DeltaPath::Kind::ChunkRecalculated ||
      DeltaPath::with_chunk_len(16).resolved_chunk_len() != 16 ||
      DeltaPath::chunk_len_on_tape(8).kind != DeltaPath::Kind::Chunk)
    fail("delta_path");
  ok("delta_path");
  // Default scale 1/√head_k_dim (path.rs:161-165).
  {
    DeltaInput in = good();
    if (std::fabs(in.resolved_scale() - 0.5) > 1e-15) fail("resolved_scale default");
    in.scale = 0.25;
    if (in.resolved_scale() != 0.25) fail("resolved_scale explicit");
    ok("resolved_scale");
  }
  // beta_gates: one per-head β as both gates, [b, s, h] → [b, s, h, 1].
  {
    auto [e, w] = beta_gates(Tensor::view(fake, {B, S, H}, DType::F32));
    if (e.dims() != std::vector<int64_t>{B, S, H, 1} || w.dims() != e.dims() ||
        e.data() != fake || w.data() != fake)
      fail("beta_gates");
    ok("beta_gates");
  }
  // The projection front-end's own checks (qkv.rs:397-401), before any device work.
  {
    QkvProjection pr;
    pr.nheads = 2;
    pr.head_k_dim = 4;
    pr.head_v_dim = 6;
    if (pr.conv_dim() != 2 * 4 + 2 * (4 + 6) || pr.write_gate_width() != 2 ||
        pr.d_in_proj() != 30)
      fail("qkv_projection widths");
    pr.write_gate = WriteGate::Channel;
    pr.n_householder = 2;
    pr.has_gate = true;
    pr.extra_channels = 3;
    if (pr.write_gate_width() != 2 * (8 + 12) || pr.d_in_proj() != 8 + 2 * 20 + 40 + 12 + 3)
      fail("qkv_projection widths (channel, u = 2)");
    ok("qkv_projection_widths");
    QkvProjection plain;
    plain.nheads = 2;
    plain.head_k_dim = 4;
    plain.head_v_dim = 6;
    expect_error("frontend_window_presence", DN_ERR_SHAPE,
                 "convolution window presence must match the block's convolution", [&] {
                   plain.forward_projected(Tensor::view(fake, {1, 3, 30}, DType::F32),
                                           Tensor::view(fake, {1, 28, 4}, DType::F32));
                 });
    expect_error("out_norm_gate_presence", DN_ERR_NULL, "OutNorm::Gated needs an output gate",
                 [&] { OutNorm{Tensor::view(fake, {6}, DType::F32)}.forward(
                           Tensor::view(fake, {2, 3, 6}, DType::F32)); });
    expect_error("frontend_projection_width", DN_ERR_SHAPE,
                 "projection: last axis must be d_in_proj = 30, got 31", [&] {
                   plain.forward_projected(Tensor::view(fake, {1, 3, 31}, DType::F32),
                                           std::nullopt);
                 });
  }
}

// ---------------------------------------------------------------------------
// Values against the oracle (float64), on the GPU.
// ---------------------------------------------------------------------------
struct Case {
  long B, S, H, K, V, ew, ww, dw;
  Vec q, k, v, e, w, g, s;
};

Case make_case(uint64_t seed, long B, long S, long H, long K, long V, long ew, long ww, long dw,
               double g_scale, double state_std, double beta_scale = 1.0) {
  Rng r(seed);
  Case c{B, S, H, K, V, ew, ww, dw, {}, {}, {}, {}, {}, {}, {}};
  const size_t rows = size_t(B * S * H);
  c.q = l2_rows(r.normals(rows * K), size_t(K));
  c.k = l2_rows(r.normals(rows * K), size_t(K));
  c.v = r.normals(rows * V);
  c.e = sigmoid(r.normals(rows * ew));
  for (auto& x : c.e) x *= beta_scale;
  c.w = ew == 1 && ww == 1 ? c.e : sigmoid(r.normals(rows * ww));
  if (dw) c.g = neg_softplus(r.normals(rows * dw), g_scale);
  c.s = r.normals(size_t(B * H * K * V), state_std);
  return c;
}

DeltaInput to_device(Case& c, DType qkv) {
  DeltaInput in{upload(c.q, {c.B, c.S, c.H, c.K}, qkv),
                upload(c.k, {c.B, c.S, c.H, c.K}, qkv),
                upload(c.v, {c.B, c.S, c.H, c.V}, qkv),
                upload(c.e, {c.B, c.S, c.H, c.ew}, DType::F32),
                upload(c.w, {c.B, c.S, c.H, c.ww}, DType::F32),
                std::nullopt,
                upload(c.s, {c.B, c.H, c.K, c.V}, DType::F32),
                std::nullopt};
  if (c.dw) in.g_bshK = upload(c.g, {c.B, c.S, c.H, c.dw}, DType::F32);
  return in;
}

std::pair<Vec, Vec> oracle_fwd(const Case& c, long L, double scale) {
  Vec y(size_t(c.B * c.S * c.H * c.V)), s(c.s.size());
  if (or_chunk_fwd_f64(c.B, c.S, c.H, c.K, c.V, c.ew, c.ww, c.dw, L, c.q.data(), c.k.data(),
                       c.v.data(), c.e.data(), c.w.data(), c.dw ? c.g.data() : nullptr,
                       c.s.data(), scale, y.data(), s.data()))
    fail("oracle chunk_fwd rejected the case");
  return {y, s};
}

void gpu_cases() {
  // B=1, H=4, T=512, dk=dv=64, chunk 64, fp32, β gates,
  // g = −softplus(N)·0.1, S₀ = 0 — through both DeltaPath arms.
  {
    Case c = make_case(20260827, 1, 512, 4, 64, 64, 1, 1, 1, 0.1, 0.0);
    DeltaInput in = to_device(c, DType::F32);
    const auto [y0, s0] = oracle_fwd(c, 64, 1.0 / 8.0);
    auto [y, s] = in.run();
    expect_close("config1_chunk_y", download(y), y0, 1e-4);
    expect_close("config1_chunk_state", download(s), s0, 1e-4);
    ok("config1_chunk");
    auto [yr, sr] = in.run(DeltaPath::recurrent());
    expect_close("config1_recurrent_y", download(yr), y0, 1e-4);
    expect_close("config1_recurrent_state", download(sr), s0, 1e-4);
    ok("config1_recurrent");
  }
  // GDN-2 gate widths (per-channel erase, write and decay), nonzero S₀,
  // a ragged last chunk, explicit scale and chunk length.
  {
    Case c = make_case(7, 2, 100, 2, 32, 48, 32, 48, 32, 0.05, 0.05);
    DeltaInput in = to_device(c, DType::F32);
    in.scale = 0.3;
    const auto [y0, s0] = oracle_fwd(c, 16, 0.3);
    auto [y, s] = in.run(DeltaPath::with_chunk_len(16));
    expect_close("channel_gates_y", download(y), y0, 1e-4);
    expect_close("channel_gates_state", download(s), s0, 1e-4);
    ok("channel_gates_chunk16");
  }
  // delta_step: out of place and in place agree, and match the oracle.
  {
    Case c = make_case(11, 3, 1, 2, 16, 24, 16, 1, 16, 0.05, 0.1);
    Vec q = c.q, k = c.k, v = c.v, e = c.e, w = c.w, g = c.g, s = c.s;
    Tensor tq = upload(q, {3, 2, 16}, DType::F32), tk = upload(k, {3, 2, 16}, DType::F32);
    Tensor tv = upload(v, {3, 2, 24}, DType::F32), te = upload(e, {3, 2, 16}, DType::F32);
    Tensor tw = upload(w, {3, 2, 1}, DType::F32), tg = upload(g, {3, 2, 16}, DType::F32);
    Tensor ts = upload(s, {3, 2, 16, 24}, DType::F32);
    Vec y0(3 * 2 * 24), s0(s.size());
    if (or_delta_step_f64(3, 2, 16, 24, 16, 1, 16, q.data(), k.data(), v.data(), e.data(),
                          w.data(), g.data(), s.data(), 0.25, y0.data(), s0.data()))
      fail("oracle delta_step rejected the case");
    auto [y, sn] = delta_step(tq, tk, tv, te, tw, tg, ts, 0.25);
    expect_close("step_y", download(y), y0, 1e-5);
    expect_close("step_state", download(sn), s0, 1e-5);
    if (rel_err(download(ts), s) != 0.0) fail("step: the input state was modified");
    Tensor yi = Tensor::empty({3, 2, 24}, DType::F32);
    delta_step_in_place(tq, tk, tv, te, tw, tg, ts, yi, 0.25);
    expect_close("step_in_place_y", download(yi), download(y), 0.0);
    expect_close("step_in_place_state", download(ts), download(sn), 0.0);
    ok("delta_step");
  }
  // combined_backward: all seven gradients at GDN-2 gate widths.
  {
    Case c = make_case(13, 1, 70, 2, 16, 24, 16, 24, 16, 0.05, 0.1);
    DeltaInput in = to_device(c, DType::F32);
    Rng r(99);
    Vec dy = r.normals(size_t(1 * 70 * 2 * 24)), dsf = r.normals(c.s.size(), 0.5);
    Tensor tdy = upload(dy, {1, 70, 2, 24}, DType::F32);
    Tensor tds = upload(dsf, {1, 2, 16, 24}, DType::F32);
    const double scale = 0.25;
    DeltaChunkGrads gr = combined_backward(tdy, tds, in.q_bshk, in.k_bshk, in.v_bshv,
                                           in.erase_bshK, in.write_bshV, in.g_bshK,
                                           in.state_bhkv, 16, scale);
    Vec dq(c.q.size()), dk(c.k.size()), dv(c.v.size()), de(c.e.size()), dw(c.w.size()),
        dg(c.g.size()), ds(c.s.size());
    if (or_chunk_bwd_f64(1, 70, 2, 16, 24, 16, 24, 16, 16, dy.data(), dsf.data(), c.q.data(),
                         c.k.data(), c.v.data(), c.e.data(), c.w.data(), c.g.data(), c.s.data(),
                         scale, dq.data(), dk.data(), dv.data(), de.data(), dw.data(), dg.data(),
                         ds.data()))
      fail("oracle chunk_bwd rejected the case");
    expect_close("bwd_dq", download(gr.d_q_bshk), dq, 1e-4);
    expect_close("bwd_dk", download(gr.d_k_bshk), dk, 1e-4);
    expect_close("bwd_dv", download(gr.d_v_bshv), dv, 1e-4);
    expect_close("bwd_derase", download(gr.d_erase_bshK), de, 1e-4);
    expect_close("bwd_dwrite", download(gr.d_write_bshV), dw, 1e-4);
    expect_close("bwd_dg", download(*gr.d_g_bshK), dg, 1e-4);
    expect_close("bwd_dstate", download(gr.d_state_bhkv), ds, 1e-4);
    ok("combined_backward");
  }
  // bf16 q/k/v at the Gated DeltaNet shape (the MFMA path), at the bf16 bar.
  {
    Case c = make_case(17, 1, 256, 2, 128, 128, 1, 1, 1, 0.05, 0.02);
    DeltaInput in = to_device(c, DType::BF16);
    const auto [y0, s0] = oracle_fwd(c, 64, 1.0 / std::sqrt(128.0));
    auto [y, s] = in.run();
    if (y.dtype() != DType::BF16) fail("bf16: y dtype");
    expect_close("bf16_y", download(y), y0, 2e-2);
    expect_close("bf16_state", download(s), s0, 2e-2);
    ok("bf16_mfma_path");
  }
  // A caller-owned Workspace: the chunk calls take their scratch from it
  // (never the library's shared pool); a larger call grows it on the stream,
  // and a later smaller one reuses it. Values as without it.
  {
    Workspace ws;
    Case c1 = make_case(19, 1, 64, 2, 128, 128, 1, 1, 1, 0.05, 0.02);
    Case c2 = make_case(23, 2, 200, 2, 128, 128, 1, 1, 1, 0.05, 0.02);
    DeltaInput in1 = to_device(c1, DType::BF16), in2 = to_device(c2, DType::BF16);
    auto [y1, s1] = in1.run(DeltaPath::chunk(), nullptr, false, &ws);
    const size_t cap1 = ws.capacity();
    if (cap1 == 0) fail("workspace: the first call reserved nothing");
    auto [y2, s2] = in2.run(DeltaPath::chunk(), nullptr, false, &ws);
    if (ws.capacity() <= cap1) fail("workspace: the larger call did not grow it");
    auto [y3, s3] = in1.run(DeltaPath::chunk(), nullptr, false, &ws);
    const auto [y10, s10] = oracle_fwd(c1, 64, 1.0 / std::sqrt(128.0));
    const auto [y20, s20] = oracle_fwd(c2, 64, 1.0 / std::sqrt(128.0));
    expect_close("workspace_y1", download(y1), y10, 2e-2);
    expect_close("workspace_y2", download(y2), y20, 2e-2);
    expect_close("workspace_s2", download(s2), s20, 2e-2);
    expect_close("workspace_y1_again", download(y3), download(y1), 0.0);
    Rng r(5);
    Vec dy = r.normals(size_t(2 * 200 * 2 * 128));
    Tensor tdy = upload(dy, {2, 200, 2, 128}, DType::BF16);
    const size_t before = ws.capacity();
    DeltaChunkGrads gr = combined_backward(tdy, std::nullopt, in2.q_bshk, in2.k_bshk,
                                           in2.v_bshv, in2.erase_bshK, in2.write_bshV,
                                           in2.g_bshK, in2.state_bhkv, 64,
                                           1.0 / std::sqrt(128.0), nullptr, false, &ws);
    if (ws.capacity() < before) fail("workspace: shrank");
    DeltaChunkGrads gd = combined_backward(tdy, std::nullopt, in2.q_bshk, in2.k_bshk,
                                           in2.v_bshv, in2.erase_bshK, in2.write_bshV,
                                           in2.g_bshK, in2.state_bhkv, 64,
                                           1.0 / std::sqrt(128.0));
    // The backward sums some gradients with atomics: equal up to their order.
    expect_close("workspace_bwd_dq", download(gr.d_q_bshk), download(gd.d_q_bshk), 1e-5);
    expect_close("workspace_bwd_dg", download(*gr.d_g_bshK), download(*gd.d_g_bshK), 1e-5);
    ok("caller_workspace");
  }
  // The projection front-end. With the newest conv tap 1 and the others 0,
  // identity activations and no norm, q and k are the raw columns, v their
  // SiLU (qkv.rs:413-421), erase 2σ and write σ of theirs (qkv.rs:356-366),
  // and the next window the last 4 raw inputs (conv.rs:108-111).
  {
    const int64_t B = 2, S = 5, H = 2, dk = 16, dv = 32, u = 2, KC = 4;
    QkvProjection pr;
    pr.nheads = H;
    pr.head_k_dim = dk;
    pr.head_v_dim = dv;
    pr.n_householder = u;
    pr.qk_activation = QkActivation::Identity;
    pr.qk_norm = QkNorm::None;
    pr.write_gate = WriteGate::Channel;
    pr.allow_neg_eigval = true;
    const int64_t cd = pr.conv_dim(), W = pr.d_in_proj(), key = H * dk, val = H * dv;
    Vec wt(size_t(cd * KC), 0.0);
    for (int64_t c = 0; c < cd; ++c) wt[size_t(c * KC + KC - 1)] = 1.0;
    pr.conv = ShortConv{upload(wt, {cd, KC}, DType::F32), std::nullopt, ConvActivation::Identity};
    Rng r(5);
    Vec raw = r.normals(size_t(B * S * W)), win = r.normals(size_t(B * cd * KC));
    Tensor tp = upload(raw, {B, S, W}, DType::F32), tw = upload(win, {B, cd, KC}, DType::F32);
    auto [o, next] = pr.forward_projected(tp, tw);
    const Vec q = download(o.q_bshk), k = download(o.k_bShk), v = download(o.v_bShv);
    const Vec e = download(o.erase_bShK), w = download(o.write_bShV), nw = download(*next);
    auto sig = [](double x) { return 1.0 / (1.0 + std::exp(-x)); };
    double err = 0.0;
    for (int64_t b = 0; b < B; ++b)
      for (int64_t t = 0; t < S; ++t) {
        const double* row = &raw[size_t((b * S + t) * W)];
        for (int64_t c = 0; c < key; ++c)
          err = std::max(err, std::fabs(q[size_t((b * S + t) * key + c)] - row[c]));
        for (int64_t c = 0; c < u * key; ++c)  // [t, m, h, :] = channel key + m·key + h·dk + :
          err = std::max(err, std::fabs(k[size_t((b * S + t) * u * key + c)] - row[key + c]));
        for (int64_t c = 0; c < u * val; ++c) {
          const double x = row[key * (1 + u) + c];
          err = std::max(err, std::fabs(v[size_t((b * S + t) * u * val + c)] - x * sig(x)));
        }
        for (int64_t c = 0; c < u * key; ++c)
          err = std::max(err, std::fabs(e[size_t((b * S + t) * u * key + c)] -
                                        2.0 * sig(row[cd + c])));
        for (int64_t c = 0; c < u * val; ++c)
          err = std::max(err, std::fabs(w[size_t((b * S + t) * u * val + c)] -
                                        sig(row[cd + u * key + c])));
      }
    for (int64_t b = 0; b < B; ++b)
      for (int64_t c = 0; c < cd; ++c)
        for (int64_t j = 0; j < KC; ++j)
          err = std::max(err, std::fabs(nw[size_t((b * cd + c) * KC + j)] -
                                        raw[size_t((b * S + S - KC + j) * W + c)]));
    if (err > 1e-5) fail("frontend closed form: max error " + std::to_string(err));
    ok("frontend_closed_form");
    // L2 norm on (qkv.rs:425-426): unit rows of q and k; and a step chain,
    // carrying the window, equals the forward.
    pr.qk_norm = QkNorm::L2;
    Vec wt2 = r.normals(size_t(cd * KC), 0.5);
    pr.conv->weight = upload(wt2, {cd, KC}, DType::F32);
    pr.conv->activation = ConvActivation::Silu;
    pr.qk_activation = QkActivation::Silu;
    auto [f, fnext] = pr.forward_projected(tp, tw);
    const Vec fq = download(f.q_bshk), fk = download(f.k_bShk);
    for (size_t row = 0; row < fq.size() / size_t(dk); ++row) {
      double n2 = 0.0;
      for (int64_t c = 0; c < dk; ++c) n2 += fq[row * size_t(dk) + size_t(c)] * fq[row * size_t(dk) + size_t(c)];
      if (std::fabs(std::sqrt(n2) - 1.0) > 1e-4) fail("frontend: q row not unit norm");
    }
    std::optional<Tensor> wcur = tw;
    for (int64_t t = 0; t < S; ++t) {
      Vec rowv(size_t(B * W));
      for (int64_t b = 0; b < B; ++b)
        for (int64_t c = 0; c < W; ++c) rowv[size_t(b * W + c)] = raw[size_t((b * S + t) * W + c)];
      auto [st, wn] = pr.step_projected(upload(rowv, {B, W}, DType::F32), wcur);
      wcur = wn;
      const Vec sq = download(st.q_bhk), sk = download(st.k_buhk);
      for (int64_t b = 0; b < B; ++b) {
        for (int64_t c = 0; c < key; ++c)
          if (std::fabs(sq[size_t(b * key + c)] - fq[size_t((b * S + t) * key + c)]) > 1e-6)
            fail("frontend: step q differs from forward");
        for (int64_t c = 0; c < u * key; ++c)
          if (std::fabs(sk[size_t(b * u * key + c)] - fk[size_t((b * S + t) * u * key + c)]) > 1e-6)
            fail("frontend: step k differs from forward");
      }
    }
    if (rel_err(download(*wcur), download(*fnext)) != 0.0) fail("frontend: step window");
    ok("frontend_step_chain");
  }
  // OutNorm on constant rows: row c with gate g gives c/√(c² + ε)·γᵢ·silu(g)
  // (norm.rs:106-113); the gate read in place from a wider projection row.
  {
    const int64_t T = 3, H = 2, D = 128, W = H * D + 10;
    Vec x(static_cast<size_t>(T * H * D)), proj(static_cast<size_t>(T * W), 0.0);
    Vec gm(static_cast<size_t>(D));
    Rng r(8);
    Vec cs = r.normals(size_t(T * H)), gs = r.normals(size_t(T * H));
    for (int64_t i = 0; i < D; ++i) gm[size_t(i)] = 0.5 + 0.01 * double(i);
    for (int64_t t = 0; t < T; ++t)
      for (int64_t h = 0; h < H; ++h)
        for (int64_t i = 0; i < D; ++i) {
          x[size_t((t * H + h) * D + i)] = cs[size_t(t * H + h)];
          proj[size_t(t * W + 3 + h * D + i)] = gs[size_t(t * H + h)];
        }
    Tensor tx = upload(x, {T, H, D}, DType::F32), tp = upload(proj, {T, W}, DType::F32);
    OutNorm norm{upload(gm, {D}, DType::F32), true, 1e-5};
    Tensor gview = Tensor::view(static_cast<float*>(tp.data()) + 3, {T, H, D}, DType::F32);
    const Vec y = download(norm.forward(tx, gview, W));
    double err = 0.0;
    for (int64_t t = 0; t < T; ++t)
      for (int64_t h = 0; h < H; ++h) {
        const double c = cs[size_t(t * H + h)], g = gs[size_t(t * H + h)];
        for (int64_t i = 0; i < D; ++i) {
          const double want = c / std::sqrt(c * c + 1e-5) * gm[size_t(i)] * g / (1.0 + std::exp(-g));
          err = std::max(err, std::fabs(y[size_t((t * H + h) * D + i)] - want));
        }
      }
    if (err > 1e-5) fail("out_norm closed form: max error " + std::to_string(err));
    ok("out_norm_closed_form");
  }
  // unit_lower_inverse of a constant-key chunk, N = −β on the strict lower
  // triangle: T[i][j] = −β(1 − β)^{i−j−1} below the diagonal (tri/tests.rs:
  // 100-128), for both solves (the series only where it is conditioned).
  for (const auto& [size, solve] : std::vector<std::pair<int64_t, TriSolve>>{
           {40, TriSolve::Blocked}, {100, TriSolve::Blocked}, {12, TriSolve::Neumann}}) {
    const double beta = 0.7;
    Vec n(size_t(2 * size * size), 0.0), want(n.size(), 0.0);
    for (int64_t b = 0; b < 2; ++b)
      for (int64_t i = 0; i < size; ++i)
        for (int64_t j = 0; j < size; ++j) {
          const size_t at = size_t((b * size + i) * size + j);
          if (j < i) {
            n[at] = -beta;
            want[at] = -beta * std::pow(1.0 - beta, double(i - j - 1));
          } else if (i == j) {
            want[at] = 1.0;
          }
        }
    const Vec t = download(unit_lower_inverse(upload(n, {2, size, size}, DType::F32), solve));
    double err = 0.0;
    for (size_t i = 0; i < t.size(); ++i) err = std::max(err, std::fabs(t[i] - want[i]));
    if (err > 1e-5)
      fail("unit_lower_inverse closed form, size " + std::to_string(size) + ": max error " +
           std::to_string(err));
  }
  ok("unit_lower_inverse_closed_form");
  // block_step (dn_block_step) equals step_projected + delta_step + OutNorm::forward
  // on the same token, fp32 throughout; the state and window updated in place.
  {
    const int64_t B = 3, H = 2, dk = 32, dv = 64, KC = 4;
    QkvProjection pr;
    pr.nheads = H;
    pr.head_k_dim = dk;
    pr.head_v_dim = dv;
    pr.has_gate = true;
    const int64_t cd = pr.conv_dim(), W = pr.d_in_proj();
    Rng r(11);
    Vec wt = r.normals(size_t(cd * KC), 0.5), raw = r.normals(size_t(B * W));
    Vec win = r.normals(size_t(B * cd * KC)), st0 = r.normals(size_t(B * H * dk * dv), 0.1);
    Vec gv(size_t(B * H), 0.0), gam(size_t(dv), 0.0);
    for (size_t i = 0; i < gv.size(); ++i) gv[i] = -0.05 * double(1 + i % 5);
    for (int64_t i = 0; i < dv; ++i) gam[size_t(i)] = 1.0 + 0.01 * double(i);
    pr.conv = ShortConv{upload(wt, {cd, KC}, DType::F32), std::nullopt, ConvActivation::Silu};
    OutNorm norm{upload(gam, {dv}, DType::F32), true, 1e-5};
    Tensor tp = upload(raw, {B, W}, DType::F32), tg = upload(gv, {B, H, 1}, DType::F32);
    const double scale = 1.0 / std::sqrt(double(dk));
    auto [st, wn] = pr.step_projected(tp, upload(win, {B, cd, KC}, DType::F32));
    auto [y, s_ref] = delta_step(st.q_bhk, st.k_buhk.reshape({B, H, dk}),
                                 st.v_buhv.reshape({B, H, dv}), st.erase_buhK.reshape({B, H, 1}),
                                 st.write_buhV.reshape({B, H, 1}), tg,
                                 upload(st0, {B, H, dk, dv}, DType::F32), scale);
    const int64_t gc = cd + pr.write_gate_width();
    Tensor zg = Tensor::view(static_cast<float*>(tp.data()) + gc, {B, H, dv}, DType::F32);
    const Vec want = download(norm.forward(y, zg, W));
    Tensor s = upload(st0, {B, H, dk, dv}, DType::F32), tw = upload(win, {B, cd, KC}, DType::F32);
    const Vec got = download(block_step(pr, norm, tp, tw, tg, s, scale));
    expect_close("block_step_out", got, want, 1e-5);
    expect_close("block_step_state", download(s), download(s_ref), 1e-5);
    if (rel_err(download(tw), download(*wn)) != 0.0) fail("block_step: window");
    ok("block_step_equals_three_calls");
  }
}

}  // namespace

int main(int argc, char** argv) {
  const bool gpu = argc > 1 && std::strcmp(argv[1], "--gpu") == 0;
  const bool host = argc > 1 && std::strcmp(argv[1], "--host-only") == 0;
  if (!gpu && !host) {
    std::fprintf(stderr, "usage: %s --host-only | --gpu\n", argv[0]);
    return 2;
  }
  try {
    host_cases();
    if (gpu) gpu_cases();
  } catch (const std::exception& e) {
    fail(std::string("unexpected exception: ") + e.what());
  }
  std::printf("all passed\n");
  return 0;
}
