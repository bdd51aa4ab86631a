// The chunkwise WY forward and its backward in fp32 arithmetic, for any
// shape, gate width and chunk length.
//
// Same three stages as the reference (src/delta/chunk_recalculated/forward.rs):
//   intra   one workgroup per chunk-head (b, n, h), fully parallel:
//           prepare (pad, scale q, in-chunk cumsum of g) → the decayed score
//           matrices → T = (I + tril(Akk,−1))⁻¹ → W = T·(ke⊙e^G), U = T·(v⊙write).
//           T comes from column-parallel forward substitution, not the
//           reference's ⌈log₂L⌉ ladder: the same inverse, L³/3 flops.
//   scan    one workgroup per (value tile, head, batch), serial over chunks:
//           V' = U − W S;  y = (q⊙e^G) S + attn V';  S ← e^{G_last}⊙S + (k⊙e^{G_last−G})ᵀ V'.
//           The value columns of S are independent, so tiles never talk.
//   bwd     (combined_backward.rs) the forward scan keeps the state entering
//           each chunk, a reverse scan keeps the state cotangent leaving each
//           chunk, and one workgroup per chunk-head then differentiates its
//           chunk in closed form (WY, score, gate and front-end terms).
// Intermediates live in a caller-sized fp32 workspace laid out per chunk-head.

#include <cmath>

#include "dn_common.hpp"

namespace dn {
namespace {

constexpr int kThreads = 256;
constexpr float kMaxExponent = 48.0f;  // src/delta/decay.rs:49

// Per-chunk-head workspace layout (float offsets).
struct Layout {
  size_t qs, kk, vv, ee, wg, gc, eg, ec, egl, ke, kg, vw, qr, kc, akk, aqk, t, w, u;
  size_t rowk, rowq, colb;  // per-channel decay: row-factor tables, one column table
  size_t per;  // floats per chunk-head
};

Layout make_layout(const Dims& d) {
  const size_t L = d.L, K = d.K, V = d.V, dwx = d.dw > 0 ? d.dw : 1;
  Layout o{};
  size_t at = 0;
  auto take = [&](size_t n) {
    size_t here = at;
    at += (n + 3) & ~size_t(3);
    return here;
  };
  o.qs = take(L * K);
  o.kk = take(L * K);
  o.vv = take(L * V);
  o.ee = take(L * d.ew);
  o.wg = take(L * d.ww);
  o.gc = take(L * dwx);
  o.eg = take(L * dwx);
  o.ec = take(L * dwx);
  o.egl = take(K);
  o.ke = take(L * K);
  o.kg = take(L * K);
  o.vw = take(L * V);
  o.qr = take(L * K);
  o.kc = take(L * K);
  o.akk = take(L * L);
  o.aqk = take(L * L);
  o.t = take(L * L);
  o.w = take(L * K);
  o.u = take(L * V);
  o.rowk = take(d.dw > 1 ? L * K : 0);
  o.rowq = take(d.dw > 1 ? L * K : 0);
  o.colb = take(d.dw > 1 ? L * K : 0);
  o.per = at;
  return o;
}

// Backward scratch per chunk-head.
struct BwdLayout {
  size_t vnew, dy, dvnew, dvw, dattn, dt, tmp, dakk, daqk, drkk, drqk, dkc, dqr, dw, dkg, dke,
      dq, dk, drke, drq, drow, drarg, dcol, degl, dgc, deg, dcarry, dgl, dref, colb;
  size_t per;
};

__host__ __device__ int decay_block_len(int L) {  // src/delta/decay.rs:55-60
  for (int m = L < 16 ? L : 16; m >= 1; --m)
    if (L % m == 0) return m;
  return 1;
}

BwdLayout make_bwd_layout(const Dims& d) {
  const size_t L = d.L, K = d.K, V = d.V, dwx = d.dw > 0 ? d.dw : 1;
  const size_t nb = d.dw > 1 ? size_t(d.L / decay_block_len(d.L)) : 1;
  BwdLayout o{};
  size_t at = 0;
  auto take = [&](size_t n) {
    size_t here = at;
    at += (n + 3) & ~size_t(3);
    return here;
  };
  o.vnew = take(L * V);
  o.dy = take(L * V);
  o.dvnew = take(L * V);
  o.dvw = take(L * V);
  o.dattn = take(L * L);
  o.dt = take(L * L);
  o.tmp = take(L * L);
  o.dakk = take(L * L);
  o.daqk = take(L * L);
  o.drkk = take(L * L);
  o.drqk = take(L * L);
  o.dkc = take(L * K);
  o.dqr = take(L * K);
  o.dw = take(L * K);
  o.dkg = take(L * K);
  o.dke = take(L * K);
  o.dq = take(L * K);
  o.dk = take(L * K);
  o.drke = take(d.dw > 1 ? L * K : 0);
  o.drq = take(d.dw > 1 ? L * K : 0);
  o.drow = take(d.dw > 1 ? L * K : 0);
  o.drarg = take(d.dw > 1 ? L * K : 0);
  o.dcol = take(d.dw > 1 ? nb * L * K : 0);
  o.degl = take(K);
  o.dgc = take(L * dwx);
  o.deg = take(L * dwx);
  o.dcarry = take(L * dwx);
  o.dgl = take(dwx);
  o.dref = take(d.dw > 1 ? nb * K : 0);
  o.colb = take(d.dw > 1 ? L * K : 0);
  o.per = at;
  return o;
}

// C (M×N) = alpha·op(A)·op(B) + beta·C over the workgroup. `tri`: 0 keeps
// every entry, 1 keeps j ≤ i, 2 keeps j < i (the rest is written as 0).
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4_t;

__device__ void wg_mm(float* C, int ldc, const float* A, int lda, bool tA, const float* B,
                      int ldb, bool tB, int M, int N, int Kd, float alpha, float beta,
                      int tri = 0) {
  if (M % 16 == 0 && N % 16 == 0 && Kd % 16 == 0 && blockDim.x % 64 == 0) {
    // On fp32 MFMA (v_mfma_f32_16x16x4_f32: fp32 products, fp32 accumulation):
    // 16×16 output tiles dealt to the waves, up to four per wave in flight
    // together (their operand reads overlap); lane l feeds A[l%16][l/16] and
    // B[l/16][l%16] of each 16×4·4×16 step and ends with D[4(l/16)+r][l%16].
    // A given (M, N) always maps an element to the same lane, so successive
    // accumulations into C need no barrier between them.
    constexpr int kTiles = 4;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6, nw = blockDim.x >> 6;
    const int m16 = lane & 15, g4 = lane >> 4;
    const int tn = N / 16, tiles = (M / 16) * tn;
    for (int t0 = wave; t0 < tiles; t0 += kTiles * nw) {
      int i0[kTiles], j0[kTiles];
      bool live[kTiles];
      f32x4_t acc[kTiles];
#pragma unroll
      for (int u = 0; u < kTiles; ++u) {
        const int t = t0 + u * nw;
        live[u] = t < tiles;
        i0[u] = live[u] ? (t / tn) * 16 : 0;
        j0[u] = live[u] ? (t % tn) * 16 : 0;
        // Tiles wholly masked by `tri` need no products.
        if ((tri == 1 && j0[u] > i0[u] + 15) || (tri == 2 && j0[u] >= i0[u] + 15)) live[u] = false;
        acc[u] = f32x4_t{0.f, 0.f, 0.f, 0.f};
      }
      for (int k0 = 0; k0 < Kd; k0 += 4) {
        const int kk = k0 + g4;
        float a[kTiles], bv[kTiles];
#pragma unroll
        for (int u = 0; u < kTiles; ++u) {
          a[u] = live[u] ? (tA ? A[size_t(kk) * lda + i0[u] + m16]
                               : A[size_t(i0[u] + m16) * lda + kk])
                         : 0.f;
          bv[u] = live[u] ? (tB ? B[size_t(j0[u] + m16) * ldb + kk]
                                : B[size_t(kk) * ldb + j0[u] + m16])
                          : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kTiles; ++u)
          acc[u] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[u], bv[u], acc[u], 0, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < kTiles; ++u) {
        const int t = t0 + u * nw;
        if (t >= tiles) continue;
        const int ti = (t / tn) * 16, tj = (t % tn) * 16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = ti + 4 * g4 + r, j = tj + m16;
          float* c = &C[size_t(i) * ldc + j];
          if ((tri == 1 && j > i) || (tri == 2 && j >= i)) {
            *c = 0.f;
          } else {
            const float prev = beta != 0.f ? beta * *c : 0.f;
            *c = alpha * acc[u][r] + prev;
          }
        }
      }
    }
    return;
  }
  for (int idx = threadIdx.x; idx < M * N; idx += blockDim.x) {
    const int i = idx / N, j = idx - i * N;
    if ((tri == 1 && j > i) || (tri == 2 && j >= i)) {
      C[size_t(i) * ldc + j] = 0.f;
      continue;
    }
    float acc = 0.f;
    for (int c = 0; c < Kd; ++c) {
      const float a = tA ? A[size_t(c) * lda + i] : A[size_t(i) * lda + c];
      const float b = tB ? B[size_t(j) * ldb + c] : B[size_t(c) * ldb + j];
      acc += a * b;
    }
    const float prev = beta != 0.f ? beta * C[size_t(i) * ldc + j] : 0.f;
    C[size_t(i) * ldc + j] = alpha * acc + prev;
  }
}

// Broadcast read of a gate laid out [L, width] at channel c.
__device__ inline float gate_at(const float* g, int width, int i, int c) {
  return g[size_t(i) * width + (width == 1 ? 0 : c)];
}

struct IntraParams {
  Dims d;
  Layout o;
  const void *q, *k, *v;
  const float *erase, *write, *g;
  float* ws;
};

// ---------------------------------------------------------------------------
// Stage 1 + 2 (forward.rs:154-332), one chunk-head per workgroup.
// ---------------------------------------------------------------------------
template <class TQ>
__global__ __launch_bounds__(kThreads) void intra_kernel(IntraParams p) {
  const Dims& d = p.d;
  const Layout& o = p.o;
  const int cid = blockIdx.x;  // ((b·N + n)·H + h)
  const int h = cid % d.H, n = (cid / d.H) % d.N, b = cid / (d.H * d.N);
  const int L = d.L, K = d.K, V = d.V, dwx = d.dw > 0 ? d.dw : 1;
  float* ws = p.ws + size_t(cid) * o.per;
  float *qs = ws + o.qs, *kk = ws + o.kk, *vv = ws + o.vv, *ee = ws + o.ee, *wg = ws + o.wg,
        *gc = ws + o.gc, *eg = ws + o.eg, *ec = ws + o.ec, *egl = ws + o.egl, *ke = ws + o.ke,
        *kg = ws + o.kg, *vw = ws + o.vw, *qr = ws + o.qr, *kc = ws + o.kc, *akk = ws + o.akk,
        *aqk = ws + o.aqk, *t = ws + o.t, *w = ws + o.w, *u = ws + o.u;
  const TQ* q = static_cast<const TQ*>(p.q);
  const TQ* k = static_cast<const TQ*>(p.k);
  const TQ* v = static_cast<const TQ*>(p.v);

  // prepare: zero pad past the sequence, q·scale (forward.rs:184-190).
  for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
    const int i = idx / K, c = idx - i * K, tok = n * L + i;
    const bool ok = tok < d.S;
    const size_t src = ((size_t(b) * d.S + tok) * d.H + h) * K + c;
    qs[idx] = ok ? ld(q, src) * d.scale : 0.f;
    kk[idx] = ok ? ld(k, src) : 0.f;
  }
  for (int idx = threadIdx.x; idx < L * V; idx += blockDim.x) {
    const int i = idx / V, c = idx - i * V, tok = n * L + i;
    vv[idx] = tok < d.S ? ld(v, ((size_t(b) * d.S + tok) * d.H + h) * V + c) : 0.f;
  }
  for (int idx = threadIdx.x; idx < L * d.ew; idx += blockDim.x) {
    const int i = idx / d.ew, c = idx - i * d.ew, tok = n * L + i;
    ee[idx] = tok < d.S ? p.erase[((size_t(b) * d.S + tok) * d.H + h) * d.ew + c] : 0.f;
  }
  for (int idx = threadIdx.x; idx < L * d.ww; idx += blockDim.x) {
    const int i = idx / d.ww, c = idx - i * d.ww, tok = n * L + i;
    wg[idx] = tok < d.S ? p.write[((size_t(b) * d.S + tok) * d.H + h) * d.ww + c] : 0.f;
  }
  // gc = in-chunk cumsum of g (forward.rs:193-194); one lane per channel.
  for (int c = threadIdx.x; c < dwx; c += blockDim.x) {
    float acc = 0.f;
    for (int i = 0; i < L; ++i) {
      const int tok = n * L + i;
      if (d.dw > 0 && tok < d.S) acc += p.g[((size_t(b) * d.S + tok) * d.H + h) * d.dw + c];
      gc[size_t(i) * dwx + c] = acc;
    }
    const float last = acc;
    for (int i = 0; i < L; ++i) {
      const float gi = gc[size_t(i) * dwx + c];
      eg[size_t(i) * dwx + c] = d.dw > 0 ? expf(gi) : 1.f;
      ec[size_t(i) * dwx + c] = d.dw > 0 ? expf(last - gi) : 1.f;
    }
  }
  __syncthreads();
  for (int c = threadIdx.x; c < K; c += blockDim.x)
    egl[c] = d.dw > 0 ? expf(gc[size_t(L - 1) * dwx + (d.dw == 1 ? 0 : c)]) : 1.f;
  for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
    const int i = idx / K, c = idx - i * K;
    const float kev = kk[idx] * gate_at(ee, d.ew, i, c);
    ke[idx] = kev;
    kg[idx] = kev * gate_at(eg, dwx, i, c);
    qr[idx] = qs[idx] * gate_at(eg, dwx, i, c);
    kc[idx] = kk[idx] * gate_at(ec, dwx, i, c);
  }
  for (int idx = threadIdx.x; idx < L * V; idx += blockDim.x) {
    const int i = idx / V, c = idx - i * V;
    vw[idx] = vv[idx] * gate_at(wg, d.ww, i, c);
  }
  __syncthreads();

  // Scores, lower triangle incl. the diagonal (forward.rs:271-318; decay.rs).
  const int mb = decay_block_len(L);
  if (d.dw > 1) {
    // Per-channel decay through the block reference point of row i's block
    // (BlockDecayPrim, forward.rs:468-556), with its clamp: the row factors
    // e^{min(G[i]−G[ref], 48)} fold into ke and q·scale once; for each row
    // block the column factors k[j]·e^{min(G[ref]−G[j], 48)} (zero for later
    // column blocks, the −∞ band) are tabulated and the block's rows of Akk
    // and Aqk are two products.
    float *rowk = ws + o.rowk, *rowq = ws + o.rowq, *colb = ws + o.colb;
    for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
      const int i = idx / K, c = idx - i * K, ref = (i / mb) * mb + mb / 2;
      const float rf =
          expf(fminf(gc[size_t(i) * dwx + c] - gc[size_t(ref) * dwx + c], kMaxExponent));
      rowk[idx] = ke[idx] * rf;
      rowq[idx] = qs[idx] * rf;
    }
    for (int pb = 0; pb < L / mb; ++pb) {
      const int ref = pb * mb + mb / 2;
      __syncthreads();  // the previous block's products are done with colb
      for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
        const int j = idx / K, c = idx - j * K;
        colb[idx] = j / mb > pb ? 0.f
                                : kk[idx] * expf(fminf(gc[size_t(ref) * dwx + c] -
                                                           gc[size_t(j) * dwx + c],
                                                       kMaxExponent));
      }
      __syncthreads();
      wg_mm(akk + size_t(pb) * mb * L, L, rowk + size_t(pb) * mb * K, K, false, colb, K, true,
            mb, L, K, 1.f, 0.f);
      wg_mm(aqk + size_t(pb) * mb * L, L, rowq + size_t(pb) * mb * K, K, false, colb, K, true,
            mb, L, K, 1.f, 0.f);
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < L * L; idx += blockDim.x) {
      const int i = idx / L, j = idx - i * L;
      if (j > i) akk[idx] = aqk[idx] = 0.f;
    }
  } else {
    for (int idx = threadIdx.x; idx < L * L; idx += blockDim.x) {
      const int i = idx / L, j = idx - i * L;
      float skk = 0.f, sqk = 0.f;
      if (j <= i) {
        for (int c = 0; c < K; ++c) {
          skk += ke[size_t(i) * K + c] * kk[size_t(j) * K + c];
          sqk += qs[size_t(i) * K + c] * kk[size_t(j) * K + c];
        }
        if (d.dw == 1) {
          const float m = expf(gc[i] - gc[j]);
          skk *= m;
          sqk *= m;
        }
      }
      akk[idx] = skk;
      aqk[idx] = sqk;  // = attn, tril(Aqk, 0) (forward.rs:255)
    }
  }
  __syncthreads();

  // T = (I + tril(Akk, −1))⁻¹: one lane per column, forward substitution.
  for (int j = threadIdx.x; j < L; j += blockDim.x) {
    for (int i = 0; i < L; ++i) t[size_t(i) * L + j] = (i == j) ? 1.f : 0.f;
    for (int i = j + 1; i < L; ++i) {
      float acc = 0.f;
      for (int c = j; c < i; ++c) acc += akk[size_t(i) * L + c] * t[size_t(c) * L + j];
      t[size_t(i) * L + j] = -acc;
    }
  }
  __syncthreads();
  // W = T (ke ⊙ e^G), U = T (v ⊙ write) (forward.rs:250-251).
  wg_mm(w, K, t, L, false, kg, K, false, L, K, L, 1.f, 0.f);
  wg_mm(u, V, t, L, false, vw, V, false, L, V, L, 1.f, 0.f);
}

// ---------------------------------------------------------------------------
// Stage 3: the serial scan (forward.rs:370-440).
// ---------------------------------------------------------------------------
struct ScanParams {
  Dims d;
  Layout o;
  int tile;          // value columns per workgroup
  const float* ws;
  const float* s_in;
  void* y;           // may be null (states-only scan)
  float* s_out;      // final state
  float* states;     // [G, K, V] state entering each chunk, or null
};

template <class TY>
__global__ __launch_bounds__(kThreads) void scan_kernel(ScanParams p) {
  const Dims& d = p.d;
  const Layout& o = p.o;
  const int h = blockIdx.y, b = blockIdx.z;
  const int j0 = blockIdx.x * p.tile;
  const int bt = min(p.tile, d.V - j0);
  const int L = d.L, K = d.K, V = d.V;
  extern __shared__ float lds[];
  float* S = lds;              // [K][tile]
  float* vn = S + K * p.tile;  // [L][tile]
  float* yb = vn + L * p.tile;  // [L][tile] (when y is written)
  const size_t bh = size_t(b) * d.H + h;

  for (int idx = threadIdx.x; idx < K * bt; idx += blockDim.x) {
    const int r = idx / bt, c = idx - r * bt;
    S[r * p.tile + c] = p.s_in[bh * K * V + size_t(r) * V + j0 + c];
  }
  __syncthreads();
  for (int n = 0; n < d.N; ++n) {
    const size_t cid = (size_t(b) * d.N + n) * d.H + h;
    const float* ws = p.ws + cid * o.per;
    const float *W = ws + o.w, *U = ws + o.u, *qr = ws + o.qr, *attn = ws + o.aqk,
                *kc = ws + o.kc, *egl = ws + o.egl;
    if (p.states)
      for (int idx = threadIdx.x; idx < K * bt; idx += blockDim.x) {
        const int r = idx / bt, c = idx - r * bt;
        p.states[cid * K * V + size_t(r) * V + j0 + c] = S[r * p.tile + c];
      }
    // V' = U − W S₀ (forward.rs:395)
    for (int idx = threadIdx.x; idx < L * bt; idx += blockDim.x) {
      const int i = idx / bt, c = idx - i * bt;
      vn[i * p.tile + c] = U[size_t(i) * V + j0 + c];
    }
    __syncthreads();
    wg_mm(vn, p.tile, W, K, false, S, p.tile, false, L, bt, K, -1.f, 1.f);
    __syncthreads();
    if (p.y) {
      // y = (Q ⊙ e^G) S₀ + attn V' (forward.rs:397-408); attn is zero above
      // its diagonal.
      wg_mm(yb, p.tile, qr, K, false, S, p.tile, false, L, bt, K, 1.f, 0.f);
      wg_mm(yb, p.tile, attn, L, false, vn, p.tile, false, L, bt, L, 1.f, 1.f);
      __syncthreads();
      for (int idx = threadIdx.x; idx < L * bt; idx += blockDim.x) {
        const int i = idx / bt, c = idx - i * bt, tok = n * L + i;
        if (tok < d.S)
          st(static_cast<TY*>(p.y), ((size_t(b) * d.S + tok) * d.H + h) * V + j0 + c,
             yb[i * p.tile + c]);
      }
    }
    // S ← S ⊙ e^{G_last} + (K ⊙ e^{G_last − G})ᵀ V' (forward.rs:412-424)
    for (int idx = threadIdx.x; idx < K * bt; idx += blockDim.x) {
      const int r = idx / bt, c = idx - r * bt;
      S[r * p.tile + c] *= egl[r];
    }
    __syncthreads();
    wg_mm(S, p.tile, kc, K, true, vn, p.tile, false, K, bt, L, 1.f, 1.f);
    __syncthreads();
  }
  for (int idx = threadIdx.x; idx < K * bt; idx += blockDim.x) {
    const int r = idx / bt, c = idx - r * bt;
    p.s_out[bh * K * V + size_t(r) * V + j0 + c] = S[r * p.tile + c];
  }
}

// ---------------------------------------------------------------------------
// Backward: the reverse scan carrying dS (combined_backward.rs:240-319, the
// dS recurrence only; every other cotangent is chunk-local).
// ---------------------------------------------------------------------------
struct RevScanParams {
  Dims d;
  Layout o;
  int tile;
  const float* ws;
  const void* dy;
  const float* dstate_final;  // may be null
  float* dstate;              // d_state output
  float* ds_after;            // [G, K, V]: state cotangent leaving each chunk
};

template <class TG>
__global__ __launch_bounds__(kThreads) void rev_scan_kernel(RevScanParams p) {
  const Dims& d = p.d;
  const Layout& o = p.o;
  const int h = blockIdx.y, b = blockIdx.z;
  const int j0 = blockIdx.x * p.tile;
  const int bt = min(p.tile, d.V - j0);
  const int L = d.L, K = d.K, V = d.V;
  extern __shared__ float lds[];
  float* dS = lds;                 // [K][tile]
  float* dvn = dS + K * p.tile;    // [L][tile]
  float* dyt = dvn + L * p.tile;   // [L][tile]
  const size_t bh = size_t(b) * d.H + h;
  const TG* dy = static_cast<const TG*>(p.dy);

  for (int idx = threadIdx.x; idx < K * bt; idx += blockDim.x) {
    const int r = idx / bt, c = idx - r * bt;
    dS[r * p.tile + c] =
        p.dstate_final ? p.dstate_final[bh * K * V + size_t(r) * V + j0 + c] : 0.f;
  }
  __syncthreads();
  for (int n = d.N - 1; n >= 0; --n) {
    const size_t cid = (size_t(b) * d.N + n) * d.H + h;
    const float* ws = p.ws + cid * o.per;
    const float *W = ws + o.w, *qr = ws + o.qr, *attn = ws + o.aqk, *kc = ws + o.kc,
                *egl = ws + o.egl;
    for (int idx = threadIdx.x; idx < K * bt; idx += blockDim.x) {
      const int r = idx / bt, c = idx - r * bt;
      p.ds_after[cid * K * V + size_t(r) * V + j0 + c] = dS[r * p.tile + c];
    }
    for (int idx = threadIdx.x; idx < L * bt; idx += blockDim.x) {
      const int i = idx / bt, c = idx - i * bt, tok = n * L + i;
      dyt[i * p.tile + c] =
          tok < d.S ? ld(dy, ((size_t(b) * d.S + tok) * d.H + h) * V + j0 + c) : 0.f;
    }
    __syncthreads();
    // dV' = attnᵀ dy + kc dS
    wg_mm(dvn, p.tile, attn, L, true, dyt, p.tile, false, L, bt, L, 1.f, 0.f);
    wg_mm(dvn, p.tile, kc, K, false, dS, p.tile, false, L, bt, K, 1.f, 1.f);
    __syncthreads();
    // dS₀ = e^{G_last} ⊙ dS + qrᵀ dy − Wᵀ dV'
    for (int idx = threadIdx.x; idx < K * bt; idx += blockDim.x) {
      const int r = idx / bt, c = idx - r * bt;
      dS[r * p.tile + c] *= egl[r];
    }
    __syncthreads();
    wg_mm(dS, p.tile, qr, K, true, dyt, p.tile, false, K, bt, L, 1.f, 1.f);
    wg_mm(dS, p.tile, W, K, true, dvn, p.tile, false, K, bt, L, -1.f, 1.f);
    __syncthreads();
  }
  for (int idx = threadIdx.x; idx < K * bt; idx += blockDim.x) {
    const int r = idx / bt, c = idx - r * bt;
    p.dstate[bh * K * V + size_t(r) * V + j0 + c] = dS[r * p.tile + c];
  }
}

// ---------------------------------------------------------------------------
// Backward: everything chunk-local, one chunk-head per workgroup
// (combined_backward.rs:240-319 per-chunk terms, :103-188, :376-513).
// ---------------------------------------------------------------------------
struct ChunkBwdParams {
  Dims d;
  Layout o;
  BwdLayout bo;
  const float* ws;
  float* bws;
  const float* states;
  const float* ds_after;
  const void* dy;
  void *dq, *dk, *dv;
  float *derase, *dwrite, *dg;
};

template <class TG>
__global__ __launch_bounds__(kThreads) void chunk_bwd_kernel(ChunkBwdParams p) {
  const Dims& d = p.d;
  const Layout& o = p.o;
  const BwdLayout& bo = p.bo;
  const int cid = blockIdx.x;
  const int h = cid % d.H, n = (cid / d.H) % d.N, b = cid / (d.H * d.N);
  const int L = d.L, K = d.K, V = d.V, dwx = d.dw > 0 ? d.dw : 1;
  const bool gated = d.dw > 0;
  const float* ws = p.ws + size_t(cid) * o.per;
  float* bw = p.bws + size_t(cid) * bo.per;
  const float *qs = ws + o.qs, *kk = ws + o.kk, *vv = ws + o.vv, *ee = ws + o.ee,
              *wg = ws + o.wg, *gc = ws + o.gc, *eg = ws + o.eg, *ec = ws + o.ec,
              *egl = ws + o.egl, *ke = ws + o.ke, *kg = ws + o.kg, *vw = ws + o.vw,
              *kc = ws + o.kc, *attn = ws + o.aqk, *T = ws + o.t,
              *W = ws + o.w, *U = ws + o.u;
  const float* S0 = p.states + size_t(cid) * K * V;
  const float* dSa = p.ds_after + size_t(cid) * K * V;
  float *vnew = bw + bo.vnew, *dyc = bw + bo.dy, *dvnew = bw + bo.dvnew, *dvw = bw + bo.dvw,
        *dattn = bw + bo.dattn, *dt = bw + bo.dt, *tmp = bw + bo.tmp, *dakk = bw + bo.dakk,
        *daqk = bw + bo.daqk, *drkk = bw + bo.drkk, *drqk = bw + bo.drqk, *dkc = bw + bo.dkc,
        *dqr = bw + bo.dqr, *dwm = bw + bo.dw, *dkg = bw + bo.dkg, *dke = bw + bo.dke,
        *dq = bw + bo.dq, *dk = bw + bo.dk, *drke = bw + bo.drke, *drq = bw + bo.drq,
        *drow = bw + bo.drow, *drarg = bw + bo.drarg, *dcol = bw + bo.dcol, *degl = bw + bo.degl, *dgc = bw + bo.dgc,
        *deg = bw + bo.deg, *dcarry = bw + bo.dcarry, *dgl = bw + bo.dgl, *dref = bw + bo.dref;
  const TG* dy = static_cast<const TG*>(p.dy);

  // V' = U − W·S₀ rebuilt, dy chunk loaded.
  for (int idx = threadIdx.x; idx < L * V; idx += blockDim.x) {
    const int i = idx / V, c = idx - i * V, tok = n * L + i;
    dyc[idx] = tok < d.S ? ld(dy, ((size_t(b) * d.S + tok) * d.H + h) * V + c) : 0.f;
    vnew[idx] = U[idx];
  }
  __syncthreads();
  wg_mm(vnew, V, W, K, false, S0, V, false, L, V, K, -1.f, 1.f);
  __syncthreads();
  // Scan cotangents of this chunk (combined_backward.rs:272-282).
  wg_mm(dattn, L, dyc, V, false, vnew, V, true, L, L, V, 1.f, 0.f);     // dy V'ᵀ
  wg_mm(dvnew, V, attn, L, true, dyc, V, false, L, V, L, 1.f, 0.f);     // attnᵀ dy
  wg_mm(dkc, K, vnew, V, false, dSa, V, true, L, K, V, 1.f, 0.f);       // V' dSᵀ
  wg_mm(dqr, K, dyc, V, false, S0, V, true, L, K, V, 1.f, 0.f);         // dy S₀ᵀ
  for (int r = threadIdx.x; r < K; r += blockDim.x) {
    float acc = 0.f;
    for (int c = 0; c < V; ++c) acc += dSa[size_t(r) * V + c] * S0[size_t(r) * V + c];
    degl[r] = acc;
  }
  __syncthreads();
  wg_mm(dvnew, V, kc, K, false, dSa, V, false, L, V, K, 1.f, 1.f);      // += kc dS
  __syncthreads();
  wg_mm(dwm, K, dvnew, V, false, S0, V, true, L, K, V, -1.f, 0.f);      // d_w = −dV' S₀ᵀ

  // Gate terms of the scan (combined_backward.rs:284-313).
  for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
    const int i = idx / K, c = idx - i * K;
    dk[idx] = dkc[idx] * gate_at(ec, dwx, i, c);
    dq[idx] = dqr[idx] * gate_at(eg, dwx, i, c);
  }
  if (gated) {
    for (int idx = threadIdx.x; idx < L * dwx; idx += blockDim.x) {
      const int i = idx / dwx, c = idx - i * dwx;
      float rk = 0.f, rq = 0.f;
      if (d.dw == 1) {
        for (int x = 0; x < K; ++x) {
          rk += dkc[size_t(i) * K + x] * kk[size_t(i) * K + x];
          rq += dqr[size_t(i) * K + x] * qs[size_t(i) * K + x];
        }
      } else {
        rk = dkc[size_t(i) * K + c] * kk[size_t(i) * K + c];
        rq = dqr[size_t(i) * K + c] * qs[size_t(i) * K + c];
      }
      dcarry[idx] = rk * ec[idx];
      deg[idx] = rq;
    }
    __syncthreads();
    for (int c = threadIdx.x; c < dwx; c += blockDim.x) {
      float acc = 0.f;
      for (int i = 0; i < L; ++i) acc += dcarry[size_t(i) * dwx + c];
      if (d.dw == 1) {
        float s = 0.f;
        for (int x = 0; x < K; ++x) s += degl[x];
        acc += s * egl[0];
      } else {
        acc += degl[c] * egl[c];
      }
      dgl[c] = acc;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < L * dwx; idx += blockDim.x) {
      const int i = idx / dwx, c = idx - i * dwx;
      dgc[idx] = -dcarry[idx] + (i == L - 1 ? dgl[c] : 0.f);
    }
  }
  __syncthreads();

  // WY backward (combined_backward.rs:103-134).
  for (int idx = threadIdx.x; idx < L * L; idx += blockDim.x) {
    const int i = idx / L, j = idx - i * L;
    daqk[idx] = j <= i ? dattn[idx] : 0.f;
  }
  wg_mm(dt, L, dvnew, V, false, vw, V, true, L, L, V, 1.f, 0.f);   // dU Vwᵀ
  wg_mm(dvw, V, T, L, true, dvnew, V, false, L, V, L, 1.f, 0.f);   // Tᵀ dU
  wg_mm(dkg, K, T, L, true, dwm, K, false, L, K, L, 1.f, 0.f);     // Tᵀ dW
  __syncthreads();
  wg_mm(dt, L, dwm, K, false, kg, K, true, L, L, K, 1.f, 1.f);     // += dW kgᵀ
  __syncthreads();
  wg_mm(tmp, L, T, L, true, dt, L, false, L, L, L, 1.f, 0.f);      // Tᵀ dT
  __syncthreads();
  wg_mm(dakk, L, tmp, L, false, T, L, true, L, L, L, -1.f, 0.f, 2);  // −tril(· Tᵀ, −1)
  for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
    const int i = idx / K, c = idx - i * K;
    dke[idx] = dkg[idx] * gate_at(eg, dwx, i, c);
  }
  __syncthreads();
  if (gated)
    for (int idx = threadIdx.x; idx < L * dwx; idx += blockDim.x) {
      const int i = idx / dwx, c = idx - i * dwx;
      float acc = 0.f;
      if (d.dw == 1)
        for (int x = 0; x < K; ++x) acc += dkg[size_t(i) * K + x] * ke[size_t(i) * K + x];
      else
        acc = dkg[size_t(i) * K + c] * ke[size_t(i) * K + c];
      deg[idx] += acc;
    }
  __syncthreads();

  // Score backward.
  const int mb = decay_block_len(L);
  if (d.dw <= 1) {
    // head_scores_backward (combined_backward.rs:376-416).
    for (int idx = threadIdx.x; idx < L * L; idx += blockDim.x) {
      const int i = idx / L, j = idx - i * L;
      const float m = gated ? (j <= i ? expf(gc[i] - gc[j]) : 0.f) : 1.f;
      drkk[idx] = dakk[idx] * m;
      drqk[idx] = daqk[idx] * m;
    }
    __syncthreads();
    wg_mm(dke, K, drkk, L, false, kk, K, false, L, K, L, 1.f, 1.f);
    wg_mm(dq, K, drqk, L, false, kk, K, false, L, K, L, 1.f, 1.f);
    wg_mm(dk, K, drkk, L, true, ke, K, false, L, K, L, 1.f, 1.f);
    __syncthreads();
    wg_mm(dk, K, drqk, L, true, qs, K, false, L, K, L, 1.f, 1.f);
    if (gated) {
      // d_diff = (dAkk ⊙ raw_kk + dAqk ⊙ raw_qk) ⊙ mask, into tmp.
      for (int idx = threadIdx.x; idx < L * L; idx += blockDim.x) {
        const int i = idx / L, j = idx - i * L;
        float val = 0.f;
        if (j <= i) {
          float rkk = 0.f, rqk = 0.f;
          for (int c = 0; c < K; ++c) {
            rkk += ke[size_t(i) * K + c] * kk[size_t(j) * K + c];
            rqk += qs[size_t(i) * K + c] * kk[size_t(j) * K + c];
          }
          val = (dakk[idx] * rkk + daqk[idx] * rqk) * expf(gc[i] - gc[j]);
        }
        tmp[idx] = val;
      }
      __syncthreads();
      for (int i = threadIdx.x; i < L; i += blockDim.x) {
        float acc = 0.f;
        for (int j = 0; j < L; ++j) acc += tmp[size_t(i) * L + j] - tmp[size_t(j) * L + i];
        dgc[i] += acc;
      }
    }
  } else {
    // channel_scores_backward (combined_backward.rs:421-513).
    const int nb = L / mb;
    auto rowf = [&](int i, int c) {
      const int ref = (i / mb) * mb + mb / 2;
      return expf(fminf(gc[size_t(i) * dwx + c] - gc[size_t(ref) * dwx + c], kMaxExponent));
    };
    auto colexp = [&](int pb, int j, int c) {
      if (j / mb > pb) return 0.f;
      const int ref = pb * mb + mb / 2;
      return expf(fminf(gc[size_t(ref) * dwx + c] - gc[size_t(j) * dwx + c], kMaxExponent));
    };
    // Per row block pb, with the column-factor table of pb:
    //   d(ke⊙rf), d(q⊙rf) rows of pb = dAkk, dAqk rows of pb · colb_pb
    //   dcol[pb] = dAkkᵀ·(ke⊙rf) + dAqkᵀ·(q⊙rf) over the rows of pb.
    const float *rowk = ws + o.rowk, *rowq = ws + o.rowq;  // written by the intra kernel
    float* colb = bw + bo.colb;
    for (int pb = 0; pb < nb; ++pb) {
      __syncthreads();  // the previous block's products are done with colb
      for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
        const int j = idx / K, c = idx - j * K;
        colb[idx] = kk[idx] * colexp(pb, j, c);
      }
      __syncthreads();
      wg_mm(drke + size_t(pb) * mb * K, K, dakk + size_t(pb) * mb * L, L, false, colb, K, false,
            mb, K, L, 1.f, 0.f);
      wg_mm(drq + size_t(pb) * mb * K, K, daqk + size_t(pb) * mb * L, L, false, colb, K, false,
            mb, K, L, 1.f, 0.f);
      wg_mm(dcol + size_t(pb) * L * K, K, dakk + size_t(pb) * mb * L, L, true,
            rowk + size_t(pb) * mb * K, K, false, L, K, mb, 1.f, 0.f);
      wg_mm(dcol + size_t(pb) * L * K, K, daqk + size_t(pb) * mb * L, L, true,
            rowq + size_t(pb) * mb * K, K, false, L, K, mb, 1.f, 1.f);
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
      const int i = idx / K, c = idx - i * K;
      const float rf = rowf(i, c);
      dke[idx] += drke[idx] * rf;
      dq[idx] += drq[idx] * rf;
      drow[idx] = drke[idx] * ke[idx] + drq[idx] * qs[idx];
    }
    // d_k from the column factor; d_gc from its exponent (clamp mask ≥ 48).
    for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
      const int j = idx / K, c = idx - j * K;
      float dkacc = 0.f, dgacc = 0.f;
      for (int pb = 0; pb < nb; ++pb) {
        const float dcv = dcol[size_t(pb) * L * K + idx];
        const float ce = colexp(pb, j, c);
        dkacc += dcv * ce;
        const int ref = pb * mb + mb / 2;
        const float e = gc[size_t(ref) * dwx + c] - gc[size_t(j) * dwx + c];
        dgacc -= (e >= kMaxExponent) ? 0.f : dcv * kk[idx] * ce;
      }
      dk[idx] += dkacc;
      dgc[idx] += dgacc;
    }
    for (int idx = threadIdx.x; idx < nb * K; idx += blockDim.x) {
      const int pb = idx / K, c = idx - pb * K, ref = pb * mb + mb / 2;
      float acc = 0.f;
      for (int j = 0; j < L; ++j) {
        const float e = gc[size_t(ref) * dwx + c] - gc[size_t(j) * dwx + c];
        acc += (e >= kMaxExponent) ? 0.f
                                   : dcol[size_t(pb) * L * K + size_t(j) * K + c] *
                                         kk[size_t(j) * K + c] * colexp(pb, j, c);
      }
      dref[idx] = acc;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
      const int i = idx / K, c = idx - i * K, ref = (i / mb) * mb + mb / 2;
      const float arg = gc[size_t(i) * dwx + c] - gc[size_t(ref) * dwx + c];
      const float dra = (arg >= kMaxExponent) ? 0.f : drow[idx] * rowf(i, c);
      drarg[idx] = dra;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < nb * K; idx += blockDim.x) {
      const int pb = idx / K, c = idx - pb * K;
      float acc = 0.f;
      for (int i = pb * mb; i < (pb + 1) * mb; ++i) acc += drarg[size_t(i) * K + c];
      dref[idx] -= acc;
    }
    __syncthreads();
    for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
      const int i = idx / K, c = idx - i * K, ref = (i / mb) * mb + mb / 2;
      dgc[idx] += drarg[idx] + (i == ref ? dref[size_t(i / mb) * K + c] : 0.f);
    }
  }
  __syncthreads();

  // Front end (combined_backward.rs:153-188) and the stores.
  for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
    const int i = idx / K, c = idx - i * K;
    dk[idx] += dke[idx] * gate_at(ee, d.ew, i, c);
  }
  if (gated)
    for (int idx = threadIdx.x; idx < L * dwx; idx += blockDim.x) dgc[idx] += deg[idx] * eg[idx];
  __syncthreads();
  if (gated)
    for (int c = threadIdx.x; c < dwx; c += blockDim.x)
      for (int i = L - 2; i >= 0; --i) dgc[size_t(i) * dwx + c] += dgc[size_t(i + 1) * dwx + c];
  __syncthreads();

  TG* gq = static_cast<TG*>(p.dq);
  TG* gk = static_cast<TG*>(p.dk);
  TG* gv = static_cast<TG*>(p.dv);
  for (int idx = threadIdx.x; idx < L * K; idx += blockDim.x) {
    const int i = idx / K, c = idx - i * K, tok = n * L + i;
    if (tok >= d.S) continue;
    const size_t dst = ((size_t(b) * d.S + tok) * d.H + h) * K + c;
    st(gq, dst, dq[idx] * d.scale);
    st(gk, dst, dk[idx]);
  }
  for (int idx = threadIdx.x; idx < L * V; idx += blockDim.x) {
    const int i = idx / V, c = idx - i * V, tok = n * L + i;
    if (tok >= d.S) continue;
    st(gv, ((size_t(b) * d.S + tok) * d.H + h) * V + c, dvw[idx] * gate_at(wg, d.ww, i, c));
  }
  for (int idx = threadIdx.x; idx < L * d.ew; idx += blockDim.x) {
    const int i = idx / d.ew, c = idx - i * d.ew, tok = n * L + i;
    if (tok >= d.S) continue;
    float acc = 0.f;
    if (d.ew == 1 && K != 1)
      for (int x = 0; x < K; ++x) acc += dke[size_t(i) * K + x] * kk[size_t(i) * K + x];
    else
      acc = dke[size_t(i) * K + c] * kk[size_t(i) * K + c];
    p.derase[((size_t(b) * d.S + tok) * d.H + h) * d.ew + c] = acc;
  }
  for (int idx = threadIdx.x; idx < L * d.ww; idx += blockDim.x) {
    const int i = idx / d.ww, c = idx - i * d.ww, tok = n * L + i;
    if (tok >= d.S) continue;
    float acc = 0.f;
    if (d.ww == 1 && V != 1)
      for (int x = 0; x < V; ++x) acc += dvw[size_t(i) * V + x] * vv[size_t(i) * V + x];
    else
      acc = dvw[size_t(i) * V + c] * vv[size_t(i) * V + c];
    p.dwrite[((size_t(b) * d.S + tok) * d.H + h) * d.ww + c] = acc;
  }
  if (gated && p.dg)
    for (int idx = threadIdx.x; idx < L * d.dw; idx += blockDim.x) {
      const int i = idx / d.dw, c = idx - i * d.dw, tok = n * L + i;
      if (tok >= d.S) continue;
      p.dg[((size_t(b) * d.S + tok) * d.H + h) * d.dw + c] = dgc[idx];
    }
}

size_t scan_lds(const Dims& d, int tile, int planes_l) {
  return sizeof(float) * size_t(tile) * (size_t(d.K) + size_t(planes_l) * d.L);
}

// Value columns per scan workgroup: 32, halved until the reverse scan's
// [K + 2L, tile] fp32 planes fit in 64 KiB of LDS.
int scan_tile(const Dims& d) {
  int tile = d.V < 32 ? d.V : 32;
  while (tile > 1 && scan_lds(d, tile, 2) > 64 * 1024) tile /= 2;
  return tile;
}

size_t G_of(const Dims& d) { return size_t(d.B) * d.N * d.H; }

}  // namespace

size_t generic_fwd_workspace(const Dims& d) {
  return align_up(G_of(d) * make_layout(d).per * sizeof(float), 256);
}

size_t generic_bwd_workspace(const Dims& d) {
  const size_t G = G_of(d);
  size_t bytes = generic_fwd_workspace(d);
  bytes += align_up(G * make_bwd_layout(d).per * sizeof(float), 256);
  bytes += 2 * align_up(G * size_t(d.K) * d.V * sizeof(float), 256);
  return bytes;
}

static hipError_t launch_intra(const Dims& d, int qkv_dtype, const void* q, const void* k,
                               const void* v, const float* erase, const float* write,
                               const float* g, float* ws, hipStream_t stream) {
  IntraParams p{d, make_layout(d), q, k, v, erase, write, g, ws};
  ProfScope ps("dn_generic_intra", stream);
  if (qkv_dtype == DN_BF16)
    hipLaunchKernelGGL(intra_kernel<bf16>, dim3(unsigned(G_of(d))), dim3(kThreads), 0, stream,
                       p);
  else
    hipLaunchKernelGGL(intra_kernel<float>, dim3(unsigned(G_of(d))), dim3(kThreads), 0, stream,
                       p);
  return hipGetLastError();
}

hipError_t generic_fwd(const Dims& d, int qkv_dtype, int y_dtype, const void* q, const void* k,
                       const void* v, const float* erase, const float* write, const float* g,
                       const float* state_in, void* y, float* state_out, void* wsv,
                       hipStream_t stream) {
  float* ws = static_cast<float*>(wsv);
  hipError_t e = launch_intra(d, qkv_dtype, q, k, v, erase, write, g, ws, stream);
  if (e != hipSuccess) return e;
  const int tile = scan_tile(d);
  ScanParams sp{d, make_layout(d), tile, ws, state_in, y, state_out, nullptr};
  dim3 grid((d.V + tile - 1) / tile, d.H, d.B);
  const size_t lds = scan_lds(d, tile, 2);  // S, V' and the y rows
  ProfScope ps("dn_generic_scan", stream);
  if (y_dtype == DN_BF16)
    hipLaunchKernelGGL(scan_kernel<bf16>, grid, dim3(kThreads), lds, stream, sp);
  else
    hipLaunchKernelGGL(scan_kernel<float>, grid, dim3(kThreads), lds, stream, sp);
  return hipGetLastError();
}

static hipError_t generic_bwd_scans(const Dims& d, int grad_dtype, const void* dy,
                                    const float* dstate_final, const float* state_in,
                                    const float* ws, float* states, float* ds_after,
                                    float* dstate, hipStream_t stream);

hipError_t generic_bwd(const Dims& d, int qkv_dtype, int grad_dtype, const void* dy,
                       const float* dstate_final, const void* q, const void* k, const void* v,
                       const float* erase, const float* write, const float* g,
                       const float* state_in, void* dq, void* dk, void* dv, float* derase,
                       float* dwrite, float* dg, float* dstate, void* wsv, hipStream_t stream,
                       void* mfma_ws) {
  const size_t G = G_of(d);
  char* base = static_cast<char*>(wsv);
  float* ws = reinterpret_cast<float*>(base);
  base += generic_fwd_workspace(d);
  float* bws = reinterpret_cast<float*>(base);
  base += align_up(G * make_bwd_layout(d).per * sizeof(float), 256);
  float* states = reinterpret_cast<float*>(base);
  base += align_up(G * size_t(d.K) * d.V * sizeof(float), 256);
  float* ds_after = reinterpret_cast<float*>(base);

  hipError_t e = launch_intra(d, qkv_dtype, q, k, v, erase, write, g, ws, stream);
  if (e != hipSuccess) return e;
  if (mfma_ws) {
    // Both scans on MFMA; the chunk-local gradients below are unchanged.
    e = mfma_bwd_scans(d, grad_dtype, dy, dstate_final, q, k, v, erase, write, g, state_in,
                       states, ds_after, dstate, mfma_ws, stream, false);
    if (e != hipSuccess) return e;
  } else if ((e = generic_bwd_scans(d, grad_dtype, dy, dstate_final, state_in, ws, states,
                                    ds_after, dstate, stream)) != hipSuccess) {
    return e;
  }
  ChunkBwdParams cp{d,     make_layout(d), make_bwd_layout(d), ws,     bws,   states,
                    ds_after, dy,           dq,                 dk,     dv,    derase,
                    dwrite,   dg};
  ProfScope ps("dn_generic_chunk_bwd", stream);
  if (grad_dtype == DN_BF16)
    hipLaunchKernelGGL(chunk_bwd_kernel<bf16>, dim3(unsigned(G)), dim3(kThreads), 0, stream, cp);
  else
    hipLaunchKernelGGL(chunk_bwd_kernel<float>, dim3(unsigned(G)), dim3(kThreads), 0, stream,
                       cp);
  return hipGetLastError();
}

static hipError_t generic_bwd_scans(const Dims& d, int grad_dtype, const void* dy,
                                    const float* dstate_final, const float* state_in,
                                    const float* ws, float* states, float* ds_after,
                                    float* dstate, hipStream_t stream) {
  hipError_t e;
  const int tile = scan_tile(d);
  dim3 grid((d.V + tile - 1) / tile, d.H, d.B);
  // Forward scan keeping the state entering each chunk; its final state goes
  // to d_state as scratch and is overwritten by the reverse scan.
  ScanParams sp{d, make_layout(d), tile, ws, state_in, nullptr, dstate, states};
  {
    ProfScope ps("dn_generic_scan_states", stream);
    hipLaunchKernelGGL(scan_kernel<float>, grid, dim3(kThreads), scan_lds(d, tile, 1), stream,
                       sp);
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  RevScanParams rp{d, make_layout(d), tile, ws, dy, dstate_final, dstate, ds_after};
  {
    ProfScope ps("dn_generic_rev_scan", stream);
    if (grad_dtype == DN_BF16)
      hipLaunchKernelGGL(rev_scan_kernel<bf16>, grid, dim3(kThreads), scan_lds(d, tile, 2),
                         stream, rp);
    else
      hipLaunchKernelGGL(rev_scan_kernel<float>, grid, dim3(kThreads), scan_lds(d, tile, 2),
                         stream, rp);
  }
  return hipGetLastError();
}

}  // namespace dn
