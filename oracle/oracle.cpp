// oracle/oracle.cpp — TEST INFRASTRUCTURE, NOT PRODUCT CODE.
//
// A CPU restatement of burn-deltanet's delta-rule core (Rust crate
// `burn-deltanet` v0.14.0, files under src/delta/), used only as the checker by
// tests/, by __graft_entry__.smoke() and as bench.py's `cpu_baseline` leg.
// Nothing in the product path links or calls this file.
//
// What it restates, function by function:
//   step<R>            src/delta/recurrent.rs:41-99        (delta_step)
//   recurrent<R>       src/delta/recurrent.rs:107-142      (DeltaInput::delta_recurrent)
//   ladder_inverse<R>  src/delta/tri/prim.rs:28-74         (Blocked unit_lower_inverse,
//                                                           the 24·L³ ladder as the reference runs it)
//   neumann_inverse<R> src/delta/tri.rs:99-107             (Neumann unit_lower_inverse: the
//                                                           series term by term, whole matrix)
//   ChunkState<R>      src/delta/chunk_recalculated/forward.rs:154-206 (Chunked::prepare)
//   wy<R>              forward.rs:235-332                  (Chunked::wy / scores / head_decay_mask / solve)
//   BlockDecay<R>      forward.rs:451-556, src/delta/decay.rs:39-60 (per-channel decay split)
//   chunk_fwd<R>       forward.rs:370-440 + chunk_recalculated.rs:115-177 (scan + default body)
//   chunk_bwd<R>       src/delta/chunk_recalculated/combined_backward.rs:72-538
//
// Pinning (see tests/): the FLA float64 fixture of src/delta/tests/reference.rs
// pins step/recurrent/chunk_fwd values for all three gate widths; the
// backward is pinned by central finite differences of `recurrent<double>` and
// by torch float64 autograd of an independent recurrence; the ladder by
// (I−N)T = I, unit-lower structure and the constant-key bound of
// src/delta/tri/tests.rs; the series by the ladder on strictly lower inputs
// and by numpy's matrix powers on a full matrix.
//
// The per-channel decay where its clamp binds (an exponent reaching
// MAX_EXPONENT = 48 within half a 16-row block, decay.rs:41-49), which no
// reference-held vector covers, is pinned by a closed form: a chunk with
// g = −10 and two orthogonal key → query pairs, one with its row exponent
// clamped and one with its column exponent clamped, whose outputs and
// gradients (a clamped exponent passes none, combined_backward.rs:480-496)
// follow by hand (tests/conftest.py, clamp_regime_case).
//
// Layouts are the reference's (src/delta/path.rs:120-141): row-major
//   q,k [B,S,H,K]  v [B,S,H,V]  erase [B,S,H,ew]  write [B,S,H,ww]
//   g [B,S,H,dw] (dw = 0: ungated)  state [B,H,K,V]  y [B,S,H,V].

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

// ---------------------------------------------------------------------------
// Dense row-major matrices and the handful of ops the core is written in.
// ---------------------------------------------------------------------------

template <class R>
struct Mat {
  long r = 0, c = 0;
  std::vector<R> d;
  Mat() = default;
  Mat(long rows, long cols) : r(rows), c(cols), d(size_t(rows * cols), R(0)) {}
  R& operator()(long i, long j) { return d[size_t(i * c + j)]; }
  const R& operator()(long i, long j) const { return d[size_t(i * c + j)]; }
};

// A·B, i-k-j order so the inner loop runs over contiguous rows.
template <class R>
Mat<R> mm(const Mat<R>& A, const Mat<R>& B) {
  Mat<R> C(A.r, B.c);
  for (long i = 0; i < A.r; ++i) {
    R* ci = &C.d[size_t(i * C.c)];
    for (long k = 0; k < A.c; ++k) {
      const R a = A(i, k);
      const R* bk = &B.d[size_t(k * B.c)];
      for (long j = 0; j < B.c; ++j) ci[j] += a * bk[j];
    }
  }
  return C;
}

template <class R>
Mat<R> tr(const Mat<R>& A) {
  Mat<R> T(A.c, A.r);
  for (long i = 0; i < A.r; ++i)
    for (long j = 0; j < A.c; ++j) T(j, i) = A(i, j);
  return T;
}

template <class R>
Mat<R> add(const Mat<R>& A, const Mat<R>& B, R sb = R(1)) {
  Mat<R> C = A;
  for (size_t i = 0; i < C.d.size(); ++i) C.d[i] += sb * B.d[i];
  return C;
}

template <class R>
Mat<R> hadamard(const Mat<R>& A, const Mat<R>& B) {
  Mat<R> C = A;
  for (size_t i = 0; i < C.d.size(); ++i) C.d[i] *= B.d[i];
  return C;
}

// `t ⊙ gate` where the gate's last axis is 1 or full (broadcast semantics of
// every gate product in forward.rs:236-237,245-247).
template <class R>
Mat<R> bmul(const Mat<R>& t, const Mat<R>& gate) {
  Mat<R> C = t;
  for (long i = 0; i < t.r; ++i)
    for (long j = 0; j < t.c; ++j) C(i, j) *= gate(i, gate.c == 1 ? 0 : j);
  return C;
}

// reduce_to_width (forward.rs:106-112): sum the last axis when the gate is 1 wide.
template <class R>
Mat<R> reduce_to_width(const Mat<R>& t, long width) {
  if (width == 1 && t.c != 1) {
    Mat<R> s(t.r, 1);
    for (long i = 0; i < t.r; ++i) {
      R acc = 0;
      for (long j = 0; j < t.c; ++j) acc += t(i, j);
      s(i, 0) = acc;
    }
    return s;
  }
  return t;
}

// tril(A, diag): keep j <= i + diag.
template <class R>
Mat<R> tril(const Mat<R>& A, long diag) {
  Mat<R> C = A;
  for (long i = 0; i < A.r; ++i)
    for (long j = 0; j < A.c; ++j)
      if (j > i + diag) C(i, j) = 0;
  return C;
}

// ---------------------------------------------------------------------------
// Problem description and tensor access.
// ---------------------------------------------------------------------------

struct Shape {
  long B, S, H, K, V;
  long ew, ww, dw;  // erase width (1|K), write width (1|V), decay width (0|1|K)
};

template <class R>
struct Inputs {
  const R *q, *k, *v, *erase, *write, *g, *state;
};

// Rows [t0, t0+rows) of a [B,S,H,width] tensor for (b,h); rows past S are the
// zero pad of forward.rs:78-85.
template <class R>
Mat<R> take(const R* x, const Shape& sh, long width, long b, long h, long t0, long rows) {
  Mat<R> m(rows, width);
  for (long i = 0; i < rows; ++i) {
    long t = t0 + i;
    if (t >= sh.S) continue;
    const R* src = x + ((b * sh.S + t) * sh.H + h) * width;
    for (long j = 0; j < width; ++j) m(i, j) = src[j];
  }
  return m;
}

template <class R>
void put(R* x, const Mat<R>& m, const Shape& sh, long width, long b, long h, long t0) {
  for (long i = 0; i < m.r; ++i) {
    long t = t0 + i;
    if (t >= sh.S) continue;
    R* dst = x + ((b * sh.S + t) * sh.H + h) * width;
    for (long j = 0; j < width; ++j) dst[j] = m(i, j);
  }
}

template <class R>
Mat<R> take_state(const R* s, const Shape& sh, long b, long h) {
  Mat<R> m(sh.K, sh.V);
  std::memcpy(m.d.data(), s + (b * sh.H + h) * sh.K * sh.V, sizeof(R) * size_t(sh.K * sh.V));
  return m;
}

template <class R>
void put_state(R* s, const Mat<R>& m, const Shape& sh, long b, long h) {
  std::memcpy(s + (b * sh.H + h) * sh.K * sh.V, m.d.data(), sizeof(R) * size_t(sh.K * sh.V));
}

// ---------------------------------------------------------------------------
// The recurrence (src/delta/recurrent.rs:41-99).
// ---------------------------------------------------------------------------

// One tick for one (b, h). `S` is updated in place; returns y.
template <class R>
std::vector<R> step_one(Mat<R>& S, const R* q, const R* k, const R* v, const R* e, long ew,
                        const R* w, long ww, const R* g, long dw, R scale) {
  const long K = S.r, V = S.c;
  // S⁻ = exp(g) ⊙ S on the key axis (recurrent.rs:57-64).
  if (dw > 0)
    for (long i = 0; i < K; ++i) {
      const R a = std::exp(g[dw == 1 ? 0 : i]);
      for (long j = 0; j < V; ++j) S(i, j) *= a;
    }
  // erased = (k ⊙ erase)ᵀ S⁻ (recurrent.rs:69-72).
  std::vector<R> u(size_t(V), R(0));
  for (long i = 0; i < K; ++i) {
    const R ke = k[i] * e[ew == 1 ? 0 : i];
    for (long j = 0; j < V; ++j) u[size_t(j)] += ke * S(i, j);
  }
  // u = v ⊙ write − erased (recurrent.rs:76).
  for (long j = 0; j < V; ++j) u[size_t(j)] = v[j] * w[ww == 1 ? 0 : j] - u[size_t(j)];
  // S = S⁻ + k uᵀ (recurrent.rs:80-83).
  for (long i = 0; i < K; ++i)
    for (long j = 0; j < V; ++j) S(i, j) += k[i] * u[size_t(j)];
  // y = (scale·q)ᵀ S (recurrent.rs:90-93).
  std::vector<R> y(size_t(V), R(0));
  for (long i = 0; i < K; ++i) {
    const R qs = q[i] * scale;
    for (long j = 0; j < V; ++j) y[size_t(j)] += qs * S(i, j);
  }
  return y;
}

template <class R>
void recurrent(const Shape& sh, const Inputs<R>& in, R scale, R* y, R* state_out) {
#pragma omp parallel for collapse(2) schedule(static)
  for (long b = 0; b < sh.B; ++b)
    for (long h = 0; h < sh.H; ++h) {
      Mat<R> S = take_state(in.state, sh, b, h);
      for (long t = 0; t < sh.S; ++t) {
        const long row = (b * sh.S + t) * sh.H + h;
        std::vector<R> yt =
            step_one(S, in.q + row * sh.K, in.k + row * sh.K, in.v + row * sh.V,
                     in.erase + row * sh.ew, sh.ew, in.write + row * sh.ww, sh.ww,
                     sh.dw > 0 ? in.g + row * sh.dw : nullptr, sh.dw, scale);
        std::memcpy(y + row * sh.V, yt.data(), sizeof(R) * size_t(sh.V));
      }
      put_state(state_out, S, sh, b, h);
    }
}

// ---------------------------------------------------------------------------
// The blocked ladder (src/delta/tri/prim.rs:28-74).
// ---------------------------------------------------------------------------

// block_strict_lower (prim.rs:55-74): 1 where ⌊i/block⌋ > ⌊j/block⌋; zeros once
// the block covers the matrix.
template <class R>
Mat<R> block_strict_lower(long size, long block) {
  Mat<R> m(size, size);
  if (block >= size) return m;
  for (long i = 0; i < size; ++i)
    for (long j = 0; j < size; ++j) m(i, j) = (i / block > j / block) ? R(1) : R(0);
  return m;
}

// T = (I − N)⁻¹ by P ← P + P X P, one level per doubling of the block
// (prim.rs:28-51).
template <class R>
Mat<R> ladder_inverse(const Mat<R>& n_strict) {
  const long size = n_strict.r;
  Mat<R> p(size, size);
  for (long i = 0; i < size; ++i) p(i, i) = 1;
  Mat<R> lower = block_strict_lower<R>(size, 1);
  long block = 1;
  while (block < size) {
    Mat<R> coarser = block_strict_lower<R>(size, block * 2);
    Mat<R> x = hadamard(n_strict, add(lower, coarser, R(-1)));
    p = add(p, mm(mm(p, x), p));
    lower = coarser;
    block *= 2;
  }
  return p;
}

// P = I + N + N² + … + N^{size−1}: term ← term·N, P ← P + term (tri.rs:99-107),
// over the whole matrix as given.
template <class R>
Mat<R> neumann_inverse(const Mat<R>& n) {
  const long size = n.r;
  Mat<R> p(size, size), term(size, size);
  for (long i = 0; i < size; ++i) p(i, i) = term(i, i) = 1;
  for (long step = 1; step < size; ++step) {
    term = mm(term, n);
    p = add(p, term);
  }
  return p;
}

// ---------------------------------------------------------------------------
// Stage 1 + 2: one chunk of one (b, h), prepared and WY-transformed.
// ---------------------------------------------------------------------------

constexpr double kMaxExponent = 48.0;  // src/delta/decay.rs:49
constexpr long kDecayBlockLen = 16;    // src/delta/decay.rs:39

// block_len (decay.rs:55-60): the largest m ≤ 16 dividing chunk_len.
long block_len(long chunk_len) {
  for (long m = std::min(kDecayBlockLen, chunk_len); m >= 1; --m)
    if (chunk_len % m == 0) return m;
  return 1;
}

template <class R>
struct Chunk {
  // Stage 1 (forward.rs:154-206): q already scaled, gc = in-chunk cumsum of g.
  Mat<R> q, k, v, e, w, gc, eg;
  // Stage 2 (forward.rs:235-266).
  Mat<R> ke, vw, kg, t, u, wm, attn;
  // Per-head decay mask (forward.rs:296-318), or the per-channel block decay
  // factors (forward.rs:468-522).
  Mat<R> mask;                       // [L, L] (gated per-head only)
  Mat<R> row;                        // [L, K] e^{min(Gᵢ − G_ref, 48)}
  std::vector<Mat<R>> col_exp, col;  // nblocks × [L, K]
  long m = 1;
};

template <class R>
Chunk<R> prepare(const Shape& sh, const Inputs<R>& in, long L, R scale, long b, long h, long n) {
  Chunk<R> c;
  const long t0 = n * L;
  c.q = take(in.q, sh, sh.K, b, h, t0, L);
  for (auto& x : c.q.d) x *= scale;
  c.k = take(in.k, sh, sh.K, b, h, t0, L);
  c.v = take(in.v, sh, sh.V, b, h, t0, L);
  c.e = take(in.erase, sh, sh.ew, b, h, t0, L);
  c.w = take(in.write, sh, sh.ww, b, h, t0, L);
  if (sh.dw > 0) {
    c.gc = take(in.g, sh, sh.dw, b, h, t0, L);
    for (long i = 1; i < L; ++i)
      for (long j = 0; j < sh.dw; ++j) c.gc(i, j) += c.gc(i - 1, j);
    c.eg = c.gc;
    for (auto& x : c.eg.d) x = std::exp(x);
  }
  return c;
}

// BlockDecayPrim::new (forward.rs:468-522).
template <class R>
void block_decay(Chunk<R>& c, long L, long K) {
  const long m = block_len(L), nb = L / m;
  c.m = m;
  c.row = Mat<R>(L, K);
  for (long i = 0; i < L; ++i) {
    const long ref = (i / m) * m + m / 2;
    for (long d = 0; d < K; ++d)
      c.row(i, d) = std::exp(std::min(c.gc(i, d) - c.gc(ref, d), R(kMaxExponent)));
  }
  c.col_exp.assign(size_t(nb), Mat<R>(L, K));
  c.col.assign(size_t(nb), Mat<R>(L, K));
  for (long p = 0; p < nb; ++p) {
    const long ref = p * m + m / 2;
    for (long j = 0; j < L; ++j)
      for (long d = 0; d < K; ++d) {
        // `−∞` band for column blocks after row block p: exactly 0.
        R ce = (j / m > p) ? R(0)
                           : std::exp(std::min(c.gc(ref, d) - c.gc(j, d), R(kMaxExponent)));
        c.col_exp[size_t(p)](j, d) = ce;
        c.col[size_t(p)](j, d) = c.k(j, d) * ce;
      }
  }
}

// BlockDecayPrim::scores (forward.rs:526-556): M[i,j] = Σ_d rowsᵢd rowᵢd col[p(i)]ⱼd.
template <class R>
Mat<R> channel_scores(const Chunk<R>& c, const Mat<R>& rows) {
  const long L = rows.r, K = rows.c;
  Mat<R> out(L, L);
  for (long i = 0; i < L; ++i) {
    const Mat<R>& col = c.col[size_t(i / c.m)];
    for (long j = 0; j < L; ++j) {
      R acc = 0;
      for (long d = 0; d < K; ++d) acc += rows(i, d) * c.row(i, d) * col(j, d);
      out(i, j) = acc;
    }
  }
  return out;
}

template <class R>
void wy(Chunk<R>& c, const Shape& sh, long L) {
  c.ke = bmul(c.k, c.e);
  c.vw = bmul(c.v, c.w);
  Mat<R> akk, aqk;
  if (sh.dw > 1) {
    block_decay(c, L, sh.K);
    akk = channel_scores(c, c.ke);
    aqk = channel_scores(c, c.q);
  } else {
    Mat<R> kT = tr(c.k);
    akk = mm(c.ke, kT);
    aqk = mm(c.q, kT);
    if (sh.dw == 1) {
      c.mask = Mat<R>(L, L);
      for (long i = 0; i < L; ++i)
        for (long j = 0; j <= i; ++j) c.mask(i, j) = std::exp(c.gc(i, 0) - c.gc(j, 0));
      akk = hadamard(akk, c.mask);
      aqk = hadamard(aqk, c.mask);
    }
  }
  // N = tril(−Akk, −1), T = (I − N)⁻¹ (forward.rs:242-243).
  Mat<R> nstrict = tril(akk, -1);
  for (auto& x : nstrict.d) x = -x;
  c.t = ladder_inverse(nstrict);
  c.kg = sh.dw > 0 ? bmul(c.ke, c.eg) : c.ke;
  c.u = mm(c.t, c.vw);
  c.wm = mm(c.t, c.kg);
  c.attn = tril(aqk, 0);
}

// The chunk-boundary carry: e^{G_last} on the state's key axis and
// k ⊙ e^{G_last − G} (forward.rs:412-424).
template <class R>
void carry_factors(const Chunk<R>& c, const Shape& sh, long L, std::vector<R>& egl, Mat<R>& ec) {
  egl.assign(size_t(sh.K), R(1));
  ec = Mat<R>(L, std::max<long>(sh.dw, 1));
  for (auto& x : ec.d) x = 1;
  if (sh.dw == 0) return;
  for (long i = 0; i < sh.K; ++i) egl[size_t(i)] = std::exp(c.gc(L - 1, sh.dw == 1 ? 0 : i));
  for (long i = 0; i < L; ++i)
    for (long j = 0; j < sh.dw; ++j) ec(i, j) = std::exp(c.gc(L - 1, j) - c.gc(i, j));
}

// ---------------------------------------------------------------------------
// Stage 3: the scan, and the trait's default body (forward.rs:370-440,
// chunk_recalculated.rs:115-177).
// ---------------------------------------------------------------------------

template <class R>
void chunk_fwd(const Shape& sh, const Inputs<R>& in, long L, R scale, R* y, R* state_out) {
  const long nchunks = (sh.S + L - 1) / L;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (long b = 0; b < sh.B; ++b)
    for (long h = 0; h < sh.H; ++h) {
      Mat<R> S = take_state(in.state, sh, b, h);
      for (long n = 0; n < nchunks; ++n) {
        Chunk<R> c = prepare(sh, in, L, scale, b, h, n);
        wy(c, sh, L);
        // V' = U − W S₀ (forward.rs:395).
        Mat<R> vnew = add(c.u, mm(c.wm, S), R(-1));
        // y = (Q ⊙ e^G) S₀ + attn V' (forward.rs:397-408).
        Mat<R> qr = sh.dw > 0 ? bmul(c.q, c.eg) : c.q;
        Mat<R> yc = add(mm(qr, S), mm(c.attn, vnew));
        put(y, yc, sh, sh.V, b, h, n * L);
        // S ← S ⊙ e^{G_last} + (K ⊙ e^{G_last − G})ᵀ V' (forward.rs:412-424).
        std::vector<R> egl;
        Mat<R> ec;
        carry_factors(c, sh, L, egl, ec);
        for (long i = 0; i < sh.K; ++i)
          for (long j = 0; j < sh.V; ++j) S(i, j) *= egl[size_t(i)];
        Mat<R> kc = sh.dw > 0 ? bmul(c.k, ec) : c.k;
        S = add(S, mm(tr(kc), vnew));
      }
      put_state(state_out, S, sh, b, h);
    }
}

// ---------------------------------------------------------------------------
// The hand-written backward (combined_backward.rs:72-538).
// ---------------------------------------------------------------------------

template <class R>
struct Grads {
  R *dq, *dk, *dv, *de, *dw, *dg, *dstate;
};

// head_scores_backward (combined_backward.rs:376-416).
template <class R>
void head_scores_backward(const Chunk<R>& c, const Shape& sh, const Mat<R>& d_akk,
                          const Mat<R>& d_aqk, Mat<R>& d_ke, Mat<R>& d_q, Mat<R>& d_k,
                          Mat<R>& d_gc) {
  const bool gated = sh.dw > 0;
  Mat<R> d_raw_kk = gated ? hadamard(d_akk, c.mask) : d_akk;
  Mat<R> d_raw_qk = gated ? hadamard(d_aqk, c.mask) : d_aqk;
  d_ke = mm(d_raw_kk, c.k);
  d_q = mm(d_raw_qk, c.k);
  d_k = add(mm(tr(d_raw_kk), c.ke), mm(tr(d_raw_qk), c.q));
  if (gated) {
    Mat<R> kT = tr(c.k);
    Mat<R> raw_kk = mm(c.ke, kT), raw_qk = mm(c.q, kT);
    Mat<R> d_mask = add(hadamard(d_akk, raw_kk), hadamard(d_aqk, raw_qk));
    Mat<R> d_diff = hadamard(d_mask, c.mask);
    const long L = d_diff.r;
    d_gc = Mat<R>(L, 1);
    for (long i = 0; i < L; ++i) {
      R acc = 0;
      for (long j = 0; j < L; ++j) acc += d_diff(i, j) - d_diff(j, i);
      d_gc(i, 0) = acc;
    }
  }
}

// channel_scores_backward (combined_backward.rs:421-513).
template <class R>
void channel_scores_backward(const Chunk<R>& c, const Shape& sh, long L, const Mat<R>& d_akk,
                             const Mat<R>& d_aqk, Mat<R>& d_ke, Mat<R>& d_q, Mat<R>& d_k,
                             Mat<R>& d_gc) {
  const long K = sh.K, m = c.m, nb = L / m;
  Mat<R> rows_ke = hadamard(c.ke, c.row), rows_q = hadamard(c.q, c.row);
  Mat<R> d_rows_ke(L, K), d_rows_q(L, K);
  std::vector<Mat<R>> d_col(size_t(nb), Mat<R>(L, K));
  for (long i = 0; i < L; ++i) {
    const long p = i / m;
    const Mat<R>& col = c.col[size_t(p)];
    for (long j = 0; j < L; ++j) {
      const R a = d_akk(i, j), b = d_aqk(i, j);
      for (long d = 0; d < K; ++d) {
        d_rows_ke(i, d) += a * col(j, d);
        d_rows_q(i, d) += b * col(j, d);
        d_col[size_t(p)](j, d) += a * rows_ke(i, d) + b * rows_q(i, d);
      }
    }
  }
  d_ke = hadamard(d_rows_ke, c.row);
  d_q = hadamard(d_rows_q, c.row);
  Mat<R> d_row = add(hadamard(d_rows_ke, c.ke), hadamard(d_rows_q, c.q));
  d_k = Mat<R>(L, K);
  d_gc = Mat<R>(L, K);
  Mat<R> d_ref(nb, K);
  for (long p = 0; p < nb; ++p) {
    const long ref = p * m + m / 2;
    for (long j = 0; j < L; ++j)
      for (long d = 0; d < K; ++d) {
        const R dc = d_col[size_t(p)](j, d), ce = c.col_exp[size_t(p)](j, d);
        d_k(j, d) += dc * ce;
        const R e = c.gc(ref, d) - c.gc(j, d);
        const R de = (e >= R(kMaxExponent)) ? R(0) : dc * c.k(j, d) * ce;
        d_ref(p, d) += de;
        d_gc(j, d) -= de;
      }
  }
  for (long i = 0; i < L; ++i) {
    const long p = i / m, ref = p * m + m / 2;
    for (long d = 0; d < K; ++d) {
      const R arg = c.gc(i, d) - c.gc(ref, d);
      const R dra = (arg >= R(kMaxExponent)) ? R(0) : d_row(i, d) * c.row(i, d);
      d_gc(i, d) += dra;
      d_ref(p, d) -= dra;
    }
  }
  for (long p = 0; p < nb; ++p)
    for (long d = 0; d < K; ++d) d_gc(p * m + m / 2, d) += d_ref(p, d);
}

template <class R>
void chunk_bwd(const Shape& sh, const Inputs<R>& in, long L, R scale, const R* dy,
               const R* dstate_final, const Grads<R>& out) {
  const long nchunks = (sh.S + L - 1) / L;
  const bool gated = sh.dw > 0;
#pragma omp parallel for collapse(2) schedule(dynamic)
  for (long b = 0; b < sh.B; ++b)
    for (long h = 0; h < sh.H; ++h) {
      // ── Recompute (combined_backward.rs:86-94): chunks and entering states.
      std::vector<Chunk<R>> cs;
      std::vector<Mat<R>> states;
      Mat<R> S = take_state(in.state, sh, b, h);
      for (long n = 0; n < nchunks; ++n) {
        Chunk<R> c = prepare(sh, in, L, scale, b, h, n);
        wy(c, sh, L);
        states.push_back(S);
        Mat<R> vnew = add(c.u, mm(c.wm, S), R(-1));
        std::vector<R> egl;
        Mat<R> ec;
        carry_factors(c, sh, L, egl, ec);
        for (long i = 0; i < sh.K; ++i)
          for (long j = 0; j < sh.V; ++j) S(i, j) *= egl[size_t(i)];
        Mat<R> kc = gated ? bmul(c.k, ec) : c.k;
        S = add(S, mm(tr(kc), vnew));
        cs.push_back(std::move(c));
      }
      // ── Reverse scan (combined_backward.rs:211-341).
      Mat<R> dS = take_state(dstate_final, sh, b, h);
      for (long n = nchunks - 1; n >= 0; --n) {
        Chunk<R>& c = cs[size_t(n)];
        const Mat<R>& S0 = states[size_t(n)];
        Mat<R> dyc = take(dy, sh, sh.V, b, h, n * L, L);
        Mat<R> S0T = tr(S0);
        Mat<R> vnew = add(c.u, mm(c.wm, S0), R(-1));
        std::vector<R> egl;
        Mat<R> ec;
        carry_factors(c, sh, L, egl, ec);
        Mat<R> kc = gated ? bmul(c.k, ec) : c.k;
        Mat<R> qr = gated ? bmul(c.q, c.eg) : c.q;

        Mat<R> d_attn = mm(dyc, tr(vnew));
        Mat<R> d_vnew = add(mm(tr(c.attn), dyc), mm(kc, dS));
        Mat<R> d_kc = mm(vnew, tr(dS));
        Mat<R> d_qr = mm(dyc, S0T);
        Mat<R> d_u = d_vnew;
        Mat<R> d_w = mm(d_vnew, S0T);
        for (auto& x : d_w.d) x = -x;
        Mat<R> dS_prev = add(mm(tr(qr), dyc), mm(tr(c.wm), d_vnew), R(-1));

        Mat<R> d_k_scan, d_q_scan, d_gc_scan, d_eg_scan;
        if (gated) {
          Mat<R> dSegl = dS;
          for (long i = 0; i < sh.K; ++i)
            for (long j = 0; j < sh.V; ++j) dSegl(i, j) *= egl[size_t(i)];
          dS_prev = add(dS_prev, dSegl);
          d_k_scan = bmul(d_kc, ec);
          Mat<R> d_carry = hadamard(reduce_to_width(hadamard(d_kc, c.k), sh.dw), ec);
          Mat<R> d_gl(1, sh.dw);
          for (long i = 0; i < L; ++i)
            for (long j = 0; j < sh.dw; ++j) d_gl(0, j) += d_carry(i, j);
          // d(S ⊙ e^{G_last}) summed back onto the gate's axis.
          std::vector<R> d_egl(size_t(sh.K), R(0));
          for (long i = 0; i < sh.K; ++i) {
            R acc = 0;
            for (long j = 0; j < sh.V; ++j) acc += dS(i, j) * S0(i, j);
            d_egl[size_t(i)] = acc;
          }
          if (sh.dw == 1) {
            R acc = 0;
            for (long i = 0; i < sh.K; ++i) acc += d_egl[size_t(i)];
            d_gl(0, 0) += acc * egl[0];
          } else {
            for (long i = 0; i < sh.K; ++i) d_gl(0, i) += d_egl[size_t(i)] * egl[size_t(i)];
          }
          d_gc_scan = d_carry;
          for (auto& x : d_gc_scan.d) x = -x;
          for (long j = 0; j < sh.dw; ++j) d_gc_scan(L - 1, j) += d_gl(0, j);
          d_eg_scan = reduce_to_width(hadamard(d_qr, c.q), sh.dw);
          d_q_scan = bmul(d_qr, c.eg);
        } else {
          dS_prev = add(dS_prev, dS);
          d_k_scan = d_kc;
          d_q_scan = d_qr;
        }
        dS = dS_prev;

        // ── WY backward (combined_backward.rs:103-134).
        Mat<R> d_aqk = tril(d_attn, 0);
        Mat<R> d_t = add(mm(d_u, tr(c.vw)), mm(d_w, tr(c.kg)));
        Mat<R> tT = tr(c.t);
        Mat<R> d_vw = mm(tT, d_u);
        Mat<R> d_kg = mm(tT, d_w);
        Mat<R> d_akk = tril(mm(mm(tT, d_t), tT), -1);
        for (auto& x : d_akk.d) x = -x;
        Mat<R> d_ke, d_eg;
        if (gated) {
          d_ke = bmul(d_kg, c.eg);
          d_eg = add(reduce_to_width(hadamard(d_kg, c.ke), sh.dw), d_eg_scan);
        } else {
          d_ke = d_kg;
        }

        // ── Scores backward (combined_backward.rs:136-151).
        Mat<R> s_ke, s_q, s_k, s_gc;
        if (sh.dw > 1)
          channel_scores_backward(c, sh, L, d_akk, d_aqk, s_ke, s_q, s_k, s_gc);
        else
          head_scores_backward(c, sh, d_akk, d_aqk, s_ke, s_q, s_k, s_gc);
        d_ke = add(d_ke, s_ke);
        Mat<R> d_q = add(d_q_scan, s_q);
        Mat<R> d_k = add(d_k_scan, s_k);

        // ── Element-wise front end (combined_backward.rs:153-188).
        d_k = add(d_k, bmul(d_ke, c.e));
        Mat<R> d_e = reduce_to_width(hadamard(d_ke, c.k), sh.ew);
        Mat<R> d_v = bmul(d_vw, c.w);
        Mat<R> d_wr = reduce_to_width(hadamard(d_vw, c.v), sh.ww);
        for (auto& x : d_q.d) x *= scale;
        put(out.dq, d_q, sh, sh.K, b, h, n * L);
        put(out.dk, d_k, sh, sh.K, b, h, n * L);
        put(out.dv, d_v, sh, sh.V, b, h, n * L);
        put(out.de, d_e, sh, sh.ew, b, h, n * L);
        put(out.dw, d_wr, sh, sh.ww, b, h, n * L);
        if (gated) {
          Mat<R> d_gc = add(d_gc_scan, s_gc);
          d_gc = add(d_gc, hadamard(d_eg, c.eg));
          // Reverse cumulative sum along the chunk.
          for (long i = L - 2; i >= 0; --i)
            for (long j = 0; j < sh.dw; ++j) d_gc(i, j) += d_gc(i + 1, j);
          put(out.dg, d_gc, sh, sh.dw, b, h, n * L);
        }
      }
      put_state(out.dstate, dS, sh, b, h);
    }
}

template <class R>
int check_shape(const Shape& sh, long L) {
  if (sh.B < 1 || sh.S < 1 || sh.H < 1 || sh.K < 1 || sh.V < 1) return -1;
  if (!(sh.ew == 1 || sh.ew == sh.K)) return -2;
  if (!(sh.ww == 1 || sh.ww == sh.V)) return -2;
  if (!(sh.dw == 0 || sh.dw == 1 || sh.dw == sh.K)) return -2;
  if (L < 1) return -3;
  return 0;
}

}  // namespace

// ---------------------------------------------------------------------------
// C entry points (called from Python through ctypes).
// ---------------------------------------------------------------------------

#define OR_SHAPE Shape sh{B, S, H, K, V, ew, ww, dw}
#define OR_DEFINE(R, SUF)                                                                      \
  extern "C" int or_delta_step_##SUF(long B, long H, long K, long V, long ew, long ww,       \
                                     long dw, const R* q, const R* k, const R* v,              \
                                     const R* erase, const R* write, const R* g,               \
                                     const R* state, R scale, R* y, R* state_out) {            \
    long S = 1;                                                                                \
    OR_SHAPE;                                                                                  \
    if (int rc = check_shape<R>(sh, 1)) return rc;                                             \
    recurrent<R>(sh, Inputs<R>{q, k, v, erase, write, g, state}, scale, y, state_out);        \
    return 0;                                                                                  \
  }                                                                                            \
  extern "C" int or_recurrent_##SUF(long B, long S, long H, long K, long V, long ew, long ww, \
                                    long dw, const R* q, const R* k, const R* v,               \
                                    const R* erase, const R* write, const R* g,                \
                                    const R* state, R scale, R* y, R* state_out) {             \
    OR_SHAPE;                                                                                  \
    if (int rc = check_shape<R>(sh, 1)) return rc;                                             \
    recurrent<R>(sh, Inputs<R>{q, k, v, erase, write, g, state}, scale, y, state_out);        \
    return 0;                                                                                  \
  }                                                                                            \
  extern "C" int or_chunk_fwd_##SUF(long B, long S, long H, long K, long V, long ew, long ww, \
                                    long dw, long L, const R* q, const R* k, const R* v,       \
                                    const R* erase, const R* write, const R* g,                \
                                    const R* state, R scale, R* y, R* state_out) {             \
    OR_SHAPE;                                                                                  \
    if (int rc = check_shape<R>(sh, L)) return rc;                                             \
    chunk_fwd<R>(sh, Inputs<R>{q, k, v, erase, write, g, state}, L, scale, y, state_out);     \
    return 0;                                                                                  \
  }                                                                                            \
  extern "C" int or_chunk_bwd_##SUF(                                                           \
      long B, long S, long H, long K, long V, long ew, long ww, long dw, long L, const R* dy,  \
      const R* dstate, const R* q, const R* k, const R* v, const R* erase, const R* write,     \
      const R* g, const R* state, R scale, R* dq, R* dk, R* dv, R* de, R* dwr, R* dg,          \
      R* dstate_out) {                                                                         \
    OR_SHAPE;                                                                                  \
    if (int rc = check_shape<R>(sh, L)) return rc;                                             \
    chunk_bwd<R>(sh, Inputs<R>{q, k, v, erase, write, g, state}, L, scale, dy, dstate,        \
                 Grads<R>{dq, dk, dv, de, dwr, dg, dstate_out});                               \
    return 0;                                                                                  \
  }                                                                                            \
  extern "C" int or_unit_lower_inverse_##SUF(long flat, long size, const R* n, R* t) {        \
    if (flat < 1 || size < 1) return -1;                                                       \
    for (long f = 0; f < flat; ++f) {                                                          \
      Mat<R> m(size, size);                                                                    \
      std::memcpy(m.d.data(), n + f * size * size, sizeof(R) * size_t(size * size));           \
      Mat<R> inv = ladder_inverse(m);                                                          \
      std::memcpy(t + f * size * size, inv.d.data(), sizeof(R) * size_t(size * size));         \
    }                                                                                          \
    return 0;                                                                                  \
  }                                                                                            \
  extern "C" int or_neumann_inverse_##SUF(long flat, long size, const R* n, R* t) {           \
    if (flat < 1 || size < 1) return -1;                                                       \
    for (long f = 0; f < flat; ++f) {                                                          \
      Mat<R> m(size, size);                                                                    \
      std::memcpy(m.d.data(), n + f * size * size, sizeof(R) * size_t(size * size));           \
      Mat<R> inv = neumann_inverse(m);                                                         \
      std::memcpy(t + f * size * size, inv.d.data(), sizeof(R) * size_t(size * size));         \
    }                                                                                          \
    return 0;                                                                                  \
  }

OR_DEFINE(float, f32)
OR_DEFINE(double, f64)

extern "C" void or_set_threads(int n) {
#ifdef _OPENMP
  omp_set_num_threads(n > 0 ? n : 1);
#else
  (void)n;
#endif
}

extern "C" int or_max_threads() {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}
