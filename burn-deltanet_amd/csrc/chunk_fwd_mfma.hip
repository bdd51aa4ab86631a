// The chunkwise WY forward on CDNA4 matrix cores (bf16 MFMA, fp32 state).
//
// Covers the per-head gate shapes of Gated DeltaNet / DeltaNet / DeltaProduct:
// bf16 q/k/v, head_k_dim ∈ {64, 128}, head_v_dim a multiple of 64,
// chunk_len 64, erase/write/forget gates of width 1 (or no forget gate);
// head_k_dim 256 with head_v_dim a multiple of 128 in the forward. The
// per-channel kernels below cover the channel-wide gates. Everything else
// takes the generic kernels.
//
// Two kernels on v_mfma_f32_16x16x32_bf16 (64-lane waves):
//
// intra  chunk-heads (b, n, h) are fully parallel; the resident workgroups
//        (two per CU) walk them, prefetching the next chunk's K/Q/gates into
//        registers. K·Kᵀ and Q·Kᵀ (the ten lower 16×16 block pairs) run on
//        MFMA with the per-head decay e^{Gᵢ−Gⱼ}, the erase gate and the
//        readout scale applied to the fp32 accumulators; T = (I + tril(Akk,
//        −1))⁻¹ is a blocked forward substitution in fp32 (four 16×16
//        diagonal blocks by column elimination, then two doubling merges
//        T₂₁ = −T₂₂ A₂₁ T₁₁ on fp32 MFMA) — the reference's ladder
//        (tri/prim.rs:28-51) at L³/3 instead of 24·L³ flops. Writes T as bf16
//        hi + lo parts, attn = tril(Aqk) as bf16 and the in-chunk cumulative
//        gate G as fp32.
//
// scan   one workgroup per (b, h, block of 16·W value columns), serial over
//        chunks; each of its W waves owns 16 value columns and all K state
//        rows, in fp32 MFMA accumulators for the whole sequence. A chunk's
//        operand tiles (K, Q, T hi/lo, attn) are staged once in LDS
//        (double-buffered: one barrier per chunk); everything that depends on
//        the state stays in the wave. Per chunk, with U − W S = T (w⊙V −
//        e⊙e^G⊙(K S)) so that neither U nor W is ever formed:
//          X  = w⊙V − (e⊙e^G)⊙(K·S)                 S as bf16 hi + lo parts
//          yᵀ = (scale·e^G)⊙(Sᵀ·Qᵀ)                 same S fragments
//          V' = T·X                                 hi + lo parts of T and X
//          yᵀ += V'ᵀ·attnᵀ;  S ← e^{G_last}⊙S + Kᵀ·(e^{G_last−G}⊙V')
//        (Kᵀ's fragments through the LDS transpose read of the K tile).
//        The contraction index of the staged tiles is permuted inside each
//        32-deep k-step so accumulator tiles serve as MFMA operands in place.

#include <algorithm>
#include <type_traits>
#include <map>
#include <mutex>

#include "activations.hpp"
#include "dn_common.hpp"
#include "mfma_scan.hpp"
#include "mfma_util.hpp"
#include "wy_inverse.hpp"

namespace dn {
namespace {

constexpr int kThreads = 256;  // 4 waves
constexpr int kBV = 64;       // head_v_dim granularity of the MFMA path

// The backward's transposed tiles. The reverse scan contracts over a chunk's
// tokens where the forward contracts over its rows, so it reads Tᵀ (hi, lo),
// attnᵀ, Kc = (Kcᵀ)ᵀ, and Qgᵀ = (scale·e^G⊙Q)ᵀ, Kgᵀ = (e⊙e^G⊙K)ᵀ
// (combined_backward.rs:272-282: the state cotangent picks up qrᵀ·dy and
// Wᵀ·dV' = kgᵀ·(Tᵀ·dV')). The intra kernels write them in their BT mode.
struct BwdTiles {
  uint16_t *Tt, *Ttl, *AtT;  // [G][64][64]
  uint16_t* Kc;              // [G][64][K]
  uint16_t *QgT, *KgT;       // [G][K][64]
  float* egl;                // [G][K] e^{G_last} per key channel
};

// ---------------------------------------------------------------------------
// intra
// ---------------------------------------------------------------------------
// Sum over each row of 16 lanes, the result in every lane of the row: the
// four DPP steps dn_frontend's L2 norm takes (pairs, quads, half rows, rows),
// in its order, so that a norm formed here equals its output bit for bit.
__device__ inline float sum16_rows(float x) {
  auto dpp = [](float v, auto ctrl) -> float {
    return __int_as_float(
        __builtin_amdgcn_update_dpp(0, __float_as_int(v), decltype(ctrl)::value, 0xF, 0xF, false));
  };
  x += dpp(x, std::integral_constant<int, 0xB1>{});   // quad_perm [1,0,3,2]
  x += dpp(x, std::integral_constant<int, 0x4E>{});   // quad_perm [2,3,0,1]
  x += dpp(x, std::integral_constant<int, 0x141>{});  // row_half_mirror
  x += dpp(x, std::integral_constant<int, 0x140>{});  // row_mirror
  return x;
}

// FE (dn_frontend_chunk_fwd): the intra kernel forms q and k itself from the
// projection, as dn_frontend does (QkvProjection::forward, qkv.rs:386-421):
// the causal depthwise conv of length 4 over the raw q/k columns, the rows
// before the sequence from the conv window (ShortConv, conv.rs:85-121), SiLU
// (the conv's and the q/k activation fused, the reference's default,
// qkv.rs:223-229), and the L2 norm over the head (norm.rs:83-90). A token row is 16 lanes × 8
// channels, dn_frontend's layout at head_k_dim 128, with its order of
// operations, so the values equal its output. They are staged for the scores
// and written to the q and k tensors, which the scan reads: the projection's
// q/k columns are read once, where dn_frontend then dn_chunk_fwd write q and
// k and read them twice. (FeParams: dn_common.hpp.)

// BT (the backward's recompute): the kernel also writes the reverse scan's
// transposed tiles (Tᵀ hi/lo, attnᵀ, Kc, Qgᵀ, Kgᵀ, e^{G_last}) from the
// tiles it holds in LDS, as the per-channel kernel does. FE: the front-end's
// q/k as above (head_k_dim 128; a grid that is a multiple of nheads, so that
// a workgroup sees one head and keeps its conv weights in LDS).
// (FE: two workgroups per CU asked of the register allocator.)
template <int K, bool GATED, bool BT = false, bool FE = false>
__global__ __launch_bounds__(kThreads, FE ? 2 : 1)
void mfma_intra_kernel(MfmaParams p, int G, BwdTiles bt, FeParams fe) {
  constexpr int KP = K + 8;                     // padded LDS row (bf16 elements)
  constexpr int KS8 = K / 8;                    // 16-byte segments per key row
  constexpr int NLD = kL * KS8 / kThreads;      // 16-byte loads per lane per tile
  constexpr int kQBytes = kL * KP * 2;
  constexpr int kSolveBytes = (kL * (kL + 1) + (kL / 2) * (kL / 2 + 1)) * 4;
  // The Q tile is dead once the scores are formed; T and the merge scratch
  // reuse its space, which keeps two workgroups per CU.
  __shared__ __attribute__((aligned(16)))
  unsigned char qsolve[kQBytes > kSolveBytes ? kQBytes : kSolveBytes];
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kL * KP];
  uint16_t* Qs = reinterpret_cast<uint16_t*>(qsolve);
  float(*Tm)[kL + 1] = reinterpret_cast<float(*)[kL + 1]>(qsolve);  // T, fp32
  float(*Xs)[kL / 2 + 1] =
      reinterpret_cast<float(*)[kL / 2 + 1]>(qsolve + kL * (kL + 1) * 4);
  __shared__ float A[kL][kL + 1];  // strict-lower Akk, fp32 (upper blocks never read)
  __shared__ __attribute__((aligned(16))) uint16_t At[kL * (kL + 8)];  // attn, bf16
  __shared__ float gcs[kL], ers[kL];
  static_assert(!FE || (K == 128 && !BT), "the fused front-end: head_k_dim 128, forward");
  // FE: thread (s, c8) owns token rows RPT·s … +RPT−1 and channels 8·c8 … +7
  // of q and k, and holds the raw rows RPT·s − 3 … for its conv taps; the
  // conv weights and bias of the head's q and k channels sit in LDS.
  constexpr int RPT = kL * KS8 / kThreads;
  constexpr int NX = FE ? RPT + 3 : 1;
  __shared__ __attribute__((aligned(16))) float few[FE ? 2 * K : 1][4];
  __shared__ float feb[FE ? 2 * K : 1];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  // attn goes out where p.attn is set (the forward; the backward's recompute
  // forms it for attnᵀ only).
  const bool attn_out = p.attn != nullptr;
  // attn's blocks above the diagonal are zero for every chunk.
  for (int idx = tid; idx < kL * kL; idx += kThreads) {
    const int i = idx / kL, j = idx % kL;
    if (j / 16 > i / 16) At[i * (kL + 8) + j] = 0;
  }

  // The workgroup walks chunk-heads cid = blockIdx.x, + gridDim.x, …; the
  // next chunk's K, Q and gates are loaded into registers while this one
  // is processed.
  uint4 kr[NLD], qr[NLD];
  uint4 xq[NX], xk[NX];
  float gr = 0.f, er = 0.f;
  auto load = [&](int cid) {
    const int h = cid % p.H, n = (cid / p.H) % p.N, b = cid / (p.H * p.N);
    if constexpr (FE) {
      // Rows clamped into the sequence, loaded together; at its start the
      // three rows before it come from the window's columns 1 … 3.
      const int s = tid / KS8, c8 = tid % KS8;
      const int qc = h * K + 8 * c8, kc = (p.H + h) * K + 8 * c8;
      const uint16_t* pb = fe.proj + size_t(b) * p.S * size_t(fe.stride);
#pragma unroll
      for (int j = 0; j < NX; ++j) {
        const int tok = min(max(n * kL + RPT * s - 3 + j, 0), p.S - 1);
        const uint16_t* src = pb + size_t(tok) * size_t(fe.stride);
        xq[j] = *reinterpret_cast<const uint4*>(src + qc);
        xk[j] = *reinterpret_cast<const uint4*>(src + kc);
      }
      if (n == 0 && s == 0) {
        const uint16_t* wb = fe.win + size_t(b) * fe.conv_dim * 4;
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          uint32_t wq[4], wk[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            wq[e] = uint32_t(wb[size_t(qc + 2 * e) * 4 + j + 1]) |
                    (uint32_t(wb[size_t(qc + 2 * e + 1) * 4 + j + 1]) << 16);
            wk[e] = uint32_t(wb[size_t(kc + 2 * e) * 4 + j + 1]) |
                    (uint32_t(wb[size_t(kc + 2 * e + 1) * 4 + j + 1]) << 16);
          }
          xq[j] = make_uint4(wq[0], wq[1], wq[2], wq[3]);
          xk[j] = make_uint4(wk[0], wk[1], wk[2], wk[3]);
        }
      }
    }
#pragma unroll
    for (int m = 0; m < (FE ? 0 : NLD); ++m) {
      const int idx = tid + kThreads * m, row = idx / KS8, c8 = idx % KS8;
      const int tok = n * kL + row;
      kr[m] = qr[m] = make_uint4(0u, 0u, 0u, 0u);
      if (tok < p.S) {
        const size_t off = ((size_t(b) * p.S + tok) * p.H + h) * K + 8 * c8;
        kr[m] = *reinterpret_cast<const uint4*>(p.k + off);
        qr[m] = *reinterpret_cast<const uint4*>(p.q + off);
      }
    }
    if (wave == 0) {
      const int tok = n * kL + lane;
      const size_t row = (size_t(b) * p.S + tok) * p.H + h;
      gr = (GATED && tok < p.S) ? p.g[row] : 0.f;
      er = tok < p.S ? p.erase[row] : 0.f;
    }
  };
  if constexpr (FE) {
    const int h = int(blockIdx.x) % p.H;
    for (int c = tid; c < 2 * K; c += kThreads) {
      const int ch = c < K ? h * K + c : (p.H + h) * K + (c - K);
      *reinterpret_cast<float4*>(few[c]) = *reinterpret_cast<const float4*>(fe.w + size_t(ch) * 4);
      feb[c] = fe.bias ? fe.bias[ch] : 0.f;
    }
    __syncthreads();
  }
  if (int(blockIdx.x) < G) load(blockIdx.x);

  // FE: q or k (g = 0, 1) of this thread's rows from the raw rows x, into the
  // LDS tile and the output tensor (rows past the sequence end: zero in the
  // tile, not stored).
  auto fe_rows = [&](const uint4 (&x)[NX], int g, uint16_t* tile, uint16_t* out, int b, int n,
                     int h) {
    const int s = tid / KS8, c8 = tid % KS8;
    float xv[NX][8];
#pragma unroll
    for (int j = 0; j < NX; ++j) {
      const uint32_t w4[4] = {x[j].x, x[j].y, x[j].z, x[j].w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[j][2 * e] = lo_f(w4[e]);
        xv[j][2 * e + 1] = hi_f(w4[e]);
      }
    }
#pragma unroll
    for (int r = 0; r < RPT; ++r) {
      float y[8], ss = 0.f;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int c = g * K + 8 * c8 + i;
        const float4 w4 = *reinterpret_cast<const float4*>(few[c]);
        float a = feb[c];
        a = fmaf(w4.x, xv[r][i], a);
        a = fmaf(w4.y, xv[r + 1][i], a);
        a = fmaf(w4.z, xv[r + 2][i], a);
        a = fmaf(w4.w, xv[r + 3][i], a);
        // The reference's default activations (SiLU in the conv, nothing
        // after it; qkv.rs:223-229), fixed at compile time as dn_frontend's
        // FSILU kernels fix them.
        a = a * sigmoidf_(a);
        y[i] = a;
        ss = fmaf(a, a, ss);
      }
      if (fe.l2) {
        const float inv = rsqrtf(sum16_rows(ss) + 1e-6f);  // norm.rs:83-90
#pragma unroll
        for (int i = 0; i < 8; ++i) y[i] *= inv;
      }
      const int row = RPT * s + r, tok = n * kL + row;
      uint4 v = make_uint4(pk_bf16(y[0], y[1]), pk_bf16(y[2], y[3]), pk_bf16(y[4], y[5]),
                           pk_bf16(y[6], y[7]));
      if (tok < p.S)
        *reinterpret_cast<uint4*>(out + ((size_t(b) * p.S + tok) * p.H + h) * K + 8 * c8) = v;
      else
        v = make_uint4(0u, 0u, 0u, 0u);
      *reinterpret_cast<uint4*>(&tile[row * KP + 8 * c8]) = v;
    }
  };

  // T (hi, lo) and attn of the previous chunk, 16 values of one row per lane:
  // their global stores are issued after the next chunk is staged, so no
  // wait on them lands at the top of the loop.
  uint4 pend[6];
  int pend_cid = -1;
  // The forward stores them packed (mfma_util.hpp: kTriTrio elements per
  // chunk-head from p.T on, the blocks above the diagonal band left out);
  // the backward's recompute (BT) and head_k_dim 256 as full [64][64] tiles
  // (tri_packed).
  auto store_pending = [&]() {
    const int row = tid / 4, c0 = 16 * (tid % 4);
    uint16_t *tp, *lp, *ap;
    if constexpr (!tri_packed(K, BT)) {
      const size_t off = size_t(pend_cid) * kL * kL + row * kL + c0;
      tp = p.T + off;
      lp = p.Tlo + off;
      ap = attn_out ? p.attn + off : nullptr;
    } else {
      const int tb = row >> 4, kk = c0 >> 5;
      if (tb < 2 && kk == 1) return;  // above the band: zero
      tp = p.T + size_t(pend_cid) * kTriTrio + tril_step(tb, kk) * kTriBlk + (row & 15) * 32 +
           (c0 & 31);
      lp = tp + kTriPacked;
      ap = tp + 2 * kTriPacked;
    }
    uint4* tdst = reinterpret_cast<uint4*>(tp);
    uint4* ldst = reinterpret_cast<uint4*>(lp);
    tdst[0] = pend[0];
    tdst[1] = pend[1];
    ldst[0] = pend[2];
    ldst[1] = pend[3];
    if (attn_out) {
      uint4* adst = reinterpret_cast<uint4*>(ap);
      adst[0] = pend[4];
      adst[1] = pend[5];
    }
  };

  // dstᵀ[d][t] = bf16(X[t][d]·rowsc(t)) for a [64][K] tile X in LDS: an item
  // is two key channels × 16 tokens, consecutive lanes taking consecutive
  // channel pairs (conflict-free column reads, one 32-bit read per token).
  auto scaled_t = [&](const uint16_t* X, uint16_t* dst, auto rowsc) {
    for (int it = tid; it < K * 2; it += kThreads) {
      const int d = 2 * (it % (K / 2)), t0 = 16 * (it / (K / 2));
      uint32_t w0[8], w1[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = t0 + 2 * e;
        const uint32_t a = *reinterpret_cast<const uint32_t*>(&X[t * KP + d]);
        const uint32_t b = *reinterpret_cast<const uint32_t*>(&X[(t + 1) * KP + d]);
        const float s0 = rowsc(t), s1 = rowsc(t + 1);
        w0[e] = pk_bf16(lo_f(a) * s0, lo_f(b) * s1);
        w1[e] = pk_bf16(hi_f(a) * s0, hi_f(b) * s1);
      }
      uint4* dst0 = reinterpret_cast<uint4*>(dst + size_t(d) * kL + t0);
      uint4* dst1 = reinterpret_cast<uint4*>(dst + size_t(d + 1) * kL + t0);
      dst0[0] = make_uint4(w0[0], w0[1], w0[2], w0[3]);
      dst0[1] = make_uint4(w0[4], w0[5], w0[6], w0[7]);
      dst1[0] = make_uint4(w1[0], w1[1], w1[2], w1[3]);
      dst1[1] = make_uint4(w1[4], w1[5], w1[6], w1[7]);
    }
  };

  for (int cid = blockIdx.x; cid < G; cid += gridDim.x) {
    if constexpr (FE) {
      const int h = cid % p.H, n = (cid / p.H) % p.N, b = cid / (p.H * p.N);
      fe_rows(xk, 1, Ks, fe.k, b, n, h);
      fe_rows(xq, 0, Qs, fe.q, b, n, h);
    } else {
#pragma unroll
      for (int m = 0; m < NLD; ++m) {
        const int idx = tid + kThreads * m, row = idx / KS8, c8 = idx % KS8;
        *reinterpret_cast<uint4*>(&Ks[row * KP + 8 * c8]) = kr[m];
        *reinterpret_cast<uint4*>(&Qs[row * KP + 8 * c8]) = qr[m];
      }
    }
    // In-chunk cumulative gate and the erase gate, one token per lane.
    if (wave == 0) {
      float gv = gr;
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float up = __shfl_up(gv, off, 64);
        if (lane >= off) gv += up;
      }
      gcs[lane] = gv;
      ers[lane] = er;
      p.gc[size_t(cid) * kL + lane] = gv;
    }
    if (pend_cid >= 0) store_pending();
    if (cid + int(gridDim.x) < G) load(cid + gridDim.x);
    __syncthreads();

    // Akk = e ⊙ (K Kᵀ) ⊙ decay (strict lower), attn = scale (Q Kᵀ) ⊙ decay:
    // the ten lower 16×16 block pairs (rb ≥ cb) are dealt to the waves 3/3/2/2.
    {
      const int r16 = lane & 15, k8 = 8 * (lane >> 4);
#pragma unroll
      for (int pi = wave; pi < 10; pi += 4) {
        const int rb = pi < 1 ? 0 : pi < 3 ? 1 : pi < 6 ? 2 : 3;
        const int cb = pi - rb * (rb + 1) / 2;
        f32x4 acck = {0.f, 0.f, 0.f, 0.f}, accq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < K / 32; ++kk) {
          const bf16x8 ak = ld8(&Ks[(16 * rb + r16) * KP + 32 * kk + k8]);
          const bf16x8 aq = ld8(&Qs[(16 * rb + r16) * KP + 32 * kk + k8]);
          const bf16x8 bk = ld8(&Ks[(16 * cb + r16) * KP + 32 * kk + k8]);
          acck = mfma16(ak, bk, acck);
          accq = mfma16(aq, bk, accq);
        }
        const int j = 16 * cb + r16;
        const float gj = gcs[j];
        float gi[4], ei[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          gi[r] = gcs[16 * rb + 4 * (lane >> 4) + r];
          ei[r] = ers[16 * rb + 4 * (lane >> 4) + r];
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * rb + 4 * (lane >> 4) + r;
          // G is non-increasing, so the exponent is ≤ 0 wherever it is kept;
          // the clamp only keeps the masked (j > i) lanes finite.
          const float e = GATED ? __expf(fminf(gi[r] - gj, 0.f)) : 1.f;
          const float decay = (j <= i) ? e : 0.f;
          const float a = ei[r] * acck[r] * decay;
          A[i][j] = (j < i) ? a : 0.f;
          At[i * (kL + 8) + j] = uint16_t(pk_bf16(p.scale * accq[r] * decay, 0.f));
        }
      }
    }
    // Qgᵀ = (scale·e^G⊙Q)ᵀ while Q is in LDS (T takes its space next); rows
    // past the sequence end are zero in the tile.
    if constexpr (BT)
      scaled_t(Qs, bt.QgT + size_t(cid) * K * kL,
               [&](int t) { return p.scale * (GATED ? __expf(gcs[t]) : 1.f); });
    __syncthreads();

    diag_inverse(A, Tm, wave, lane);
    {
      // The backward's Kgᵀ = (e⊙e^G⊙K)ᵀ, Kc = e^{G_last−G}⊙K row-major and
      // e^{G_last} per key channel, while the K tile is in LDS. (The scan
      // reads Kᵀ from its own K tile.)
      if constexpr (BT) {
        const float glast = gcs[kL - 1];
        auto kcs = [&](int t) { return GATED ? __expf(glast - gcs[t]) : 1.f; };
        scaled_t(Ks, bt.KgT + size_t(cid) * K * kL,
                 [&](int t) { return ers[t] * (GATED ? __expf(gcs[t]) : 1.f); });
        for (int idx = tid; idx < kL * KS8; idx += kThreads) {
          const int t = idx / KS8, d0 = 8 * (idx % KS8);
          const uint4 x = *reinterpret_cast<const uint4*>(&Ks[t * KP + d0]);
          const float sc = kcs(t);
          *reinterpret_cast<uint4*>(bt.Kc + (size_t(cid) * kL + t) * K + d0) =
              make_uint4(pk_bf16(lo_f(x.x) * sc, hi_f(x.x) * sc),
                         pk_bf16(lo_f(x.y) * sc, hi_f(x.y) * sc),
                         pk_bf16(lo_f(x.z) * sc, hi_f(x.z) * sc),
                         pk_bf16(lo_f(x.w) * sc, hi_f(x.w) * sc));
        }
        const float egl = GATED ? __expf(glast) : 1.f;
        for (int d = tid; d < K; d += kThreads) bt.egl[size_t(cid) * K + d] = egl;
      }
      // Zero T above the block diagonal (the merges never write there).
      for (int idx = tid; idx < kL * kL; idx += kThreads) {
        const int i = idx / kL, j = idx % kL;
        if (j / 16 > i / 16) Tm[i][j] = 0.f;
      }
    }
    __syncthreads();
    merge_T(A, Tm, Xs, wave, lane, [] { __syncthreads(); });

    // T and attn of this chunk as bf16 rows, 16 values per lane.
    {
      const int row = tid / 4, c0 = 16 * (tid % 4);
      uint32_t tv[8], tl[8];
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float x0 = Tm[row][c0 + 2 * c], x1 = Tm[row][c0 + 2 * c + 1];
        tv[c] = pk_bf16(x0, x1);
        tl[c] = pk_bf16(x0 - lo_f(tv[c]), x1 - hi_f(tv[c]));
      }
      pend[0] = make_uint4(tv[0], tv[1], tv[2], tv[3]);
      pend[1] = make_uint4(tv[4], tv[5], tv[6], tv[7]);
      pend[2] = make_uint4(tl[0], tl[1], tl[2], tl[3]);
      pend[3] = make_uint4(tl[4], tl[5], tl[6], tl[7]);
      pend[4] = *reinterpret_cast<const uint4*>(&At[row * (kL + 8) + c0]);
      pend[5] = *reinterpret_cast<const uint4*>(&At[row * (kL + 8) + c0 + 8]);
      pend_cid = cid;
      if constexpr (BT) {
        // Tᵀ (hi, lo) and attnᵀ row `row` = column `row` of T and attn.
        uint32_t av[8];
#pragma unroll
        for (int c = 0; c < 8; ++c) {
          const int i0 = c0 + 2 * c;
          const float x0 = Tm[i0][row], x1 = Tm[i0 + 1][row];
          tv[c] = pk_bf16(x0, x1);
          tl[c] = pk_bf16(x0 - lo_f(tv[c]), x1 - hi_f(tv[c]));
          av[c] = uint32_t(At[i0 * (kL + 8) + row]) | (uint32_t(At[(i0 + 1) * (kL + 8) + row]) << 16);
        }
        const size_t off = size_t(cid) * kL * kL + row * kL + c0;
        uint4* ttd = reinterpret_cast<uint4*>(bt.Tt + off);
        uint4* tld = reinterpret_cast<uint4*>(bt.Ttl + off);
        uint4* atd = reinterpret_cast<uint4*>(bt.AtT + off);
        ttd[0] = make_uint4(tv[0], tv[1], tv[2], tv[3]);
        ttd[1] = make_uint4(tv[4], tv[5], tv[6], tv[7]);
        tld[0] = make_uint4(tl[0], tl[1], tl[2], tl[3]);
        tld[1] = make_uint4(tl[4], tl[5], tl[6], tl[7]);
        atd[0] = make_uint4(av[0], av[1], av[2], av[3]);
        atd[1] = make_uint4(av[4], av[5], av[6], av[7]);
      }
    }
    __syncthreads();  // LDS is restaged by the next chunk
  }
  if (pend_cid >= 0) store_pending();
}

// ---------------------------------------------------------------------------
// intra, per-channel gates (GDN-2: decay of width K, erase of width 1 or K)
// ---------------------------------------------------------------------------
// The scores follow the reference's block decay (decay.rs:39-60,
// forward.rs:451-556): for the 16-row block holding row i, with reference row
// r = 16·(i div 16) + 8,
//   Akk[i][j] = Σ_d (k⊙e)[i][d]·e^{min(G[i][d]−G[r][d], 48)} · k[j][d]·e^{min(G[r][d]−G[j][d], 48)}
// (j < i; Aqk likewise with scale·q and j ≤ i). The row factors are formed
// one 16-row block at a time as bf16 tiles (hi + lo for Akk, which feeds the
// inverse); the column factors, which depend on the row block, are formed per
// MFMA fragment in registers. Besides T/attn/Kcᵀ the kernel writes what the scan
// needs in place of K, Q and the scalar gates: kg = e⊙e^G⊙K (hi + lo),
// qg = scale·e^G⊙Q and e^{G_last} per channel. One workgroup per chunk-head.
// BT (the backward's recompute): the kernel also writes the reverse scan's
// transposed tiles (Tᵀ hi/lo, attnᵀ, Kc, Qgᵀ, Kgᵀ, e^{G_last}), the same
// values the transposing pass of the per-head backward produces. EW1: the
// erase gate has width 1 (else K). HD: the forget gate is per head (width 1,
// or none) while the erase or write gate is per channel (WriteGate::Channel
// blocks of Gated DeltaNet / DeltaNet): G is the same in every channel, and
// the scores take the reference's head mask e^{Gᵢ−Gⱼ} (head_decay_mask,
// forward.rs:290-312) on the fp32 accumulators in place of the block factors,
// so the block decay's clamp (a per-channel device) never applies.
template <int K, bool BT, bool EW1, bool HD = false>
__global__ __launch_bounds__(kThreads) void mfma_intra_pc_kernel(MfmaParams p, BwdTiles bt) {
  constexpr int GP = K + 4;  // fp32 row pitch of G
  constexpr int KS8 = K / 8;
  constexpr int NLD = kL * KS8 / kThreads;
  constexpr int NIT = 16 * KS8;  // items (one row, 8 channels) of a 16-row block
  static_assert(NIT <= kThreads, "one item per thread per row block");
  constexpr int kGBytes = kL * GP * 4;
  constexpr int kSolveBytes = (kL * (kL + 1) + (kL / 2) * (kL / 2 + 1)) * 4;
  constexpr float kMaxExp = 48.f;  // MAX_EXPONENT, decay.rs:49
  // K rows and the row-factor tiles are unpadded: a row's 16-byte segments
  // are permuted by its row index, so the 16 rows an MFMA operand read spans
  // cover 16 distinct 16-byte bank slots (rows of 128 bytes pair up per 256
  // bytes, hence the shift when K = 64).
  constexpr int kSwz = KS8 >= 16 ? 0 : 1;
  auto sw = [](int row, int col) {
    return row * K + ((((col >> 3) ^ (row >> kSwz)) & (KS8 - 1)) << 3) + (col & 7);
  };
  // 79 KB at K = 128, which keeps two workgroups per CU: the row-factor
  // tiles hold one 16-row block at a time, attn goes to memory straight from
  // the accumulators, and T with the merge scratch takes G's place once Kcᵀ
  // is written.
  __shared__ __attribute__((aligned(16))) uint16_t Ks[kL * K];
  __shared__ __attribute__((aligned(16)))
  unsigned char gsolve[kGBytes > kSolveBytes ? kGBytes : kSolveBytes];
  __shared__ __attribute__((aligned(16))) uint16_t RT[3][16 * K];  // (k⊙e)·rf hi, lo; scale·q·rf
  __shared__ float A[kL][kL + 1];  // strict-lower Akk, fp32 (upper blocks never read)
  float* Gc = reinterpret_cast<float*>(gsolve);
  float(*Tm)[kL + 1] = reinterpret_cast<float(*)[kL + 1]>(gsolve);
  float(*Xs)[kL / 2 + 1] = reinterpret_cast<float(*)[kL / 2 + 1]>(gsolve + kL * (kL + 1) * 4);

  const int cid = blockIdx.x;
  const int h = cid % p.H, n = (cid / p.H) % p.N, b = cid / (p.H * p.N);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tok0 = n * kL;
  const size_t row0 = size_t(b) * p.S * p.H + h + size_t(tok0) * p.H;
  const int valid = min(kL, p.S - tok0);
  auto row_of = [&](int t) { return row0 + size_t(t) * p.H; };
  // Global reads are unconditional: a row past the sequence end reads the
  // chunk's last row and the value is dropped (a load under a lane guard
  // becomes a branch with a full wait, which serialises the loads).
  auto rowc = [&](int t) { return row_of(min(t, valid - 1)); };
  auto f8 = [](const uint4& u, float* f) {
    f[0] = lo_f(u.x); f[1] = hi_f(u.x); f[2] = lo_f(u.y); f[3] = hi_f(u.y);
    f[4] = lo_f(u.z); f[5] = hi_f(u.z); f[6] = lo_f(u.w); f[7] = hi_f(u.w);
  };

  // K tile to LDS (zero past the sequence end): all loads first, then the
  // stores.
  uint4 kx[NLD];
#pragma unroll
  for (int m = 0; m < NLD; ++m) {
    const int idx = tid + kThreads * m, row = idx / KS8, c8 = idx % KS8;
    kx[m] = *reinterpret_cast<const uint4*>(p.k + rowc(row) * K + 8 * c8);
  }
  // This thread's item of each row block rb is row 16·rb + irow, channels
  // d0i…d0i+7: its Q segment and erase gate, in registers.
  const bool item = tid < NIT;
  const int irow = tid / KS8, d0i = 8 * (tid % KS8);
  uint4 qr[4];
  float ef[4][8];
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int i = 16 * rb + irow;
    const bool ok = item && i < valid;
    const uint4 qx = *reinterpret_cast<const uint4*>(p.q + rowc(i) * K + d0i);
    qr[rb] = ok ? qx : make_uint4(0u, 0u, 0u, 0u);
    if constexpr (EW1) {
      const float e = p.erase[rowc(i)];
#pragma unroll
      for (int x = 0; x < 8; ++x) ef[rb][x] = ok ? e : 0.f;
    } else {
      float e8[8];
      *reinterpret_cast<float4*>(e8) = *reinterpret_cast<const float4*>(p.erase + rowc(i) * K + d0i);
      *reinterpret_cast<float4*>(e8 + 4) =
          *reinterpret_cast<const float4*>(p.erase + rowc(i) * K + d0i + 4);
#pragma unroll
      for (int x = 0; x < 8; ++x) ef[rb][x] = ok ? e8[x] : 0.f;
    }
  }
  // G = in-chunk cumulative sum of g per channel: KPART lanes per channel,
  // each summing a run of tokens, then the runs' totals are carried over.
  // Its loads go out with the others, before the K tile's stores.
  constexpr int KPART = kThreads / K, RUN = kL / KPART;
  float vals[RUN];
  {
    const int d = tid % K, part = tid / K;
#pragma unroll
    for (int t = 0; t < RUN; ++t) {
      const int tt = part * RUN + t;
      float x;
      if constexpr (HD) {
        // Width 1 (or no forget gate: a valid row read and dropped, with no
        // branch around the load).
        x = (p.gated ? p.g : p.erase)[rowc(tt)];
        if (!p.gated) x = 0.f;
      } else {
        x = p.g[rowc(tt) * K + d];
      }
      vals[t] = tt < valid ? x : 0.f;
    }
  }
#pragma unroll
  for (int m = 0; m < NLD; ++m) {
    const int idx = tid + kThreads * m, row = idx / KS8, c8 = idx % KS8;
    *reinterpret_cast<uint4*>(&Ks[sw(row, 8 * c8)]) =
        row < valid ? kx[m] : make_uint4(0u, 0u, 0u, 0u);
  }
  {
    const int d = tid % K, part = tid / K;
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < RUN; ++t) {
      acc += vals[t];
      vals[t] = acc;
    }
    if (KPART > 1) Gc[(part * RUN + RUN - 1) * GP + d] = acc;
    __syncthreads();
    float carry = 0.f;
    for (int pp = 0; pp < part; ++pp) carry += Gc[(pp * RUN + RUN - 1) * GP + d];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < RUN; ++t) Gc[(part * RUN + t) * GP + d] = vals[t] + carry;
  }
  __syncthreads();

  const int r16 = lane & 15, q4 = lane >> 4, k8 = 8 * q4;
#pragma unroll
  for (int rb = 0; rb < 4; ++rb) {
    const int r = 16 * rb + 8;  // the block's reference row
    // Row factors e^{min(G[i]−G[r], 48)} of block rb into the A-operand
    // tiles, and the scan's kg / qg (e^G ≤ 1: G ≤ 0).
    if (item) {
      const int i = 16 * rb + irow;
      float gi[8], gr[8], kf[8], qf[8];
      *reinterpret_cast<float4*>(gi) = *reinterpret_cast<const float4*>(&Gc[i * GP + d0i]);
      *reinterpret_cast<float4*>(gi + 4) = *reinterpret_cast<const float4*>(&Gc[i * GP + d0i + 4]);
      *reinterpret_cast<float4*>(gr) = *reinterpret_cast<const float4*>(&Gc[r * GP + d0i]);
      *reinterpret_cast<float4*>(gr + 4) = *reinterpret_cast<const float4*>(&Gc[r * GP + d0i + 4]);
      f8(*reinterpret_cast<const uint4*>(&Ks[sw(i, d0i)]), kf);
      f8(qr[rb], qf);
      float ak[8], aq[8], kg[8], qg[8];
#pragma unroll
      for (int x = 0; x < 8; ++x) {
        const float rf = HD ? 1.f : __expf(fminf(gi[x] - gr[x], kMaxExp));
        const float eg = __expf(gi[x]);
        const float ke = kf[x] * ef[rb][x], qs = qf[x] * p.scale;
        ak[x] = ke * rf;
        aq[x] = qs * rf;
        kg[x] = ke * eg;
        qg[x] = qs * eg;
      }
      uint32_t ah[4], al[4], qh[4], gh[4], gl[4], qq[4];
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        ah[x] = pk_bf16(ak[2 * x], ak[2 * x + 1]);
        al[x] = pk_bf16(ak[2 * x] - lo_f(ah[x]), ak[2 * x + 1] - hi_f(ah[x]));
        qh[x] = pk_bf16(aq[2 * x], aq[2 * x + 1]);
        gh[x] = pk_bf16(kg[2 * x], kg[2 * x + 1]);
        gl[x] = pk_bf16(kg[2 * x] - lo_f(gh[x]), kg[2 * x + 1] - hi_f(gh[x]));
        qq[x] = pk_bf16(qg[2 * x], qg[2 * x + 1]);
      }
      const int at = sw(irow, d0i);
      *reinterpret_cast<uint4*>(&RT[0][at]) = make_uint4(ah[0], ah[1], ah[2], ah[3]);
      *reinterpret_cast<uint4*>(&RT[1][at]) = make_uint4(al[0], al[1], al[2], al[3]);
      *reinterpret_cast<uint4*>(&RT[2][at]) = make_uint4(qh[0], qh[1], qh[2], qh[3]);
      const size_t go = (size_t(cid) * kL + i) * K + d0i;
      *reinterpret_cast<uint4*>(p.Kg + go) = make_uint4(gh[0], gh[1], gh[2], gh[3]);
      *reinterpret_cast<uint4*>(p.Kglo + go) = make_uint4(gl[0], gl[1], gl[2], gl[3]);
      // qg feeds only the forward's y (the backward's scans read Qgᵀ).
      if constexpr (!BT) *reinterpret_cast<uint4*>(p.Qg + go) = make_uint4(qq[0], qq[1], qq[2], qq[3]);
      if constexpr (BT) {
        // Qgᵀ and Kgᵀ: the four lanes holding rows i0…i0+3 of the same eight
        // channels trade channel-pair words, so that lane q ends with channels
        // d0i + 2q and d0i + 2q + 1 of all four rows and stores 8 bytes for
        // each. Round s receives row (q + s) mod 4.
        const int q = (lane / KS8) & 3, lbase = lane - q * KS8;
        const int i0 = 16 * rb + (irow & ~3);
        uint32_t rq[4], rk[4];
#pragma unroll
        for (int s4 = 0; s4 < 4; ++s4) {
          const int sel = (q - s4) & 3;
          const uint32_t sq = sel == 0 ? qq[0] : sel == 1 ? qq[1] : sel == 2 ? qq[2] : qq[3];
          const uint32_t sk = sel == 0 ? gh[0] : sel == 1 ? gh[1] : sel == 2 ? gh[2] : gh[3];
          const int src = lbase + KS8 * ((q + s4) & 3);
          rq[s4] = uint32_t(__shfl(int(sq), src, 64));
          rk[s4] = uint32_t(__shfl(int(sk), src, 64));
        }
        // Rotate so that index t holds row t (t = (q + s) mod 4).
        auto rot = [&](uint32_t (&r)[4]) {
          if (q & 1) {
            const uint32_t t = r[3];
            r[3] = r[2]; r[2] = r[1]; r[1] = r[0]; r[0] = t;
          }
          if (q & 2) {
            uint32_t t = r[0]; r[0] = r[2]; r[2] = t;
            t = r[1]; r[1] = r[3]; r[3] = t;
          }
        };
        rot(rq);
        rot(rk);
        auto put = [&](uint16_t* dst, const uint32_t (&r)[4]) {
          const size_t o = (size_t(cid) * K + d0i + 2 * q) * kL + i0;
          *reinterpret_cast<uint2*>(dst + o) =
              make_uint2((r[0] & 0xffffu) | (r[1] << 16), (r[2] & 0xffffu) | (r[3] << 16));
          *reinterpret_cast<uint2*>(dst + o + kL) =
              make_uint2((r[0] >> 16) | (r[1] & 0xffff0000u), (r[2] >> 16) | (r[3] & 0xffff0000u));
        };
        put(bt.QgT, rq);
        put(bt.KgT, rk);
      }
    }
    __syncthreads();
    // Scores of block row rb: wave w ≤ rb forms block (rb, w); a wave past
    // the diagonal writes attn's zero block (rb, w). attn row i, column j:
    // the 16 lanes of one q4 store 16 consecutive columns. (The backward
    // writes attnᵀ only: attn feeds the forward's y.)
    {
      const int cb = wave, j = 16 * cb + r16;
      uint16_t* adst = BT ? nullptr : p.attn + size_t(cid) * kL * kL + size_t(16 * rb + 4 * q4) * kL + j;
      if (cb <= rb) {
        f32x4 acck = {0.f, 0.f, 0.f, 0.f}, accq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < K / 32; ++kk) {
          const int d0 = 32 * kk + k8;
          float kf[8], gj[8], gr[8];
          f8(*reinterpret_cast<const uint4*>(&Ks[sw(j, d0)]), kf);
          *reinterpret_cast<float4*>(gj) = *reinterpret_cast<const float4*>(&Gc[j * GP + d0]);
          *reinterpret_cast<float4*>(gj + 4) = *reinterpret_cast<const float4*>(&Gc[j * GP + d0 + 4]);
          *reinterpret_cast<float4*>(gr) = *reinterpret_cast<const float4*>(&Gc[r * GP + d0]);
          *reinterpret_cast<float4*>(gr + 4) = *reinterpret_cast<const float4*>(&Gc[r * GP + d0 + 4]);
          float c[8];
#pragma unroll
          for (int x = 0; x < 8; ++x)
            c[x] = HD ? kf[x] : kf[x] * __expf(fminf(gr[x] - gj[x], kMaxExp));
          uint4 bh, bl;
          bh.x = pk_bf16(c[0], c[1]);
          bh.y = pk_bf16(c[2], c[3]);
          bh.z = pk_bf16(c[4], c[5]);
          bh.w = pk_bf16(c[6], c[7]);
          bl.x = pk_bf16(c[0] - lo_f(bh.x), c[1] - hi_f(bh.x));
          bl.y = pk_bf16(c[2] - lo_f(bh.y), c[3] - hi_f(bh.y));
          bl.z = pk_bf16(c[4] - lo_f(bh.z), c[5] - hi_f(bh.z));
          bl.w = pk_bf16(c[6] - lo_f(bh.w), c[7] - hi_f(bh.w));
          const bf16x8 b_h = __builtin_bit_cast(bf16x8, bh), b_l = __builtin_bit_cast(bf16x8, bl);
          const int at = sw(r16, d0);
          const bf16x8 a_h = ld8(&RT[0][at]);
          acck = mfma16(a_h, b_h, acck);
          acck = mfma16(ld8(&RT[1][at]), b_h, acck);
          if constexpr (!HD) acck = mfma16(a_h, b_l, acck);  // HD: K is exact in bf16
          accq = mfma16(ld8(&RT[2][at]), b_h, accq);
        }
        if constexpr (HD) {
          // The head mask e^{Gᵢ−Gⱼ} (≤ 1 where kept; clamped at 0 above the
          // diagonal, which the masks below drop).
          const float gjv = Gc[j * GP];
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) {
            const float dm = __expf(fminf(Gc[(16 * rb + 4 * q4 + rr) * GP] - gjv, 0.f));
            acck[rr] *= dm;
            accq[rr] *= dm;
          }
        }
        uint32_t av[4];
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int i = 16 * rb + 4 * q4 + rr;
          A[i][j] = (j < i) ? acck[rr] : 0.f;
          av[rr] = pk_bf16((j <= i) ? accq[rr] : 0.f, 0.f);
          if constexpr (!BT) adst[rr * kL] = uint16_t(av[rr]);
        }
        if constexpr (BT)  // attnᵀ row j, columns 16·rb + 4·q4 … +3
          *reinterpret_cast<uint2*>(bt.AtT + size_t(cid) * kL * kL + size_t(j) * kL + 16 * rb +
                                    4 * q4) =
              make_uint2(av[0] | (av[1] << 16), av[2] | (av[3] << 16));
      } else {
        if constexpr (!BT) {
#pragma unroll
          for (int rr = 0; rr < 4; ++rr) adst[rr * kL] = 0;
        }
        if constexpr (BT)
          *reinterpret_cast<uint2*>(bt.AtT + size_t(cid) * kL * kL + size_t(j) * kL + 16 * rb +
                                    4 * q4) = make_uint2(0u, 0u);
      }
    }
    if (rb < 3) __syncthreads();  // the next block rewrites RT
  }

  // Kcᵀ = (e^{G_last−G}⊙K)ᵀ, two channels per item; e^{G_last}.
  for (int it = tid; it < K * 2; it += kThreads) {
    const int d = 2 * (it % (K / 2)), t0 = 16 * (it / (K / 2));
    const float gl0 = Gc[(kL - 1) * GP + d], gl1 = Gc[(kL - 1) * GP + d + 1];
    uint32_t w0[8], w1[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int t = t0 + 2 * e;
      const uint32_t a = *reinterpret_cast<const uint32_t*>(&Ks[sw(t, d)]);
      const uint32_t c = *reinterpret_cast<const uint32_t*>(&Ks[sw(t + 1, d)]);
      const float2 ga = *reinterpret_cast<const float2*>(&Gc[t * GP + d]);
      const float2 gb = *reinterpret_cast<const float2*>(&Gc[(t + 1) * GP + d]);
      w0[e] = pk_bf16(lo_f(a) * __expf(gl0 - ga.x), lo_f(c) * __expf(gl0 - gb.x));
      w1[e] = pk_bf16(hi_f(a) * __expf(gl1 - ga.y), hi_f(c) * __expf(gl1 - gb.y));
    }
    uint4* dst0 = reinterpret_cast<uint4*>(p.KcT + (size_t(cid) * K + d) * kL + t0);
    uint4* dst1 = reinterpret_cast<uint4*>(p.KcT + (size_t(cid) * K + d + 1) * kL + t0);
    dst0[0] = make_uint4(w0[0], w0[1], w0[2], w0[3]);
    dst0[1] = make_uint4(w0[4], w0[5], w0[6], w0[7]);
    dst1[0] = make_uint4(w1[0], w1[1], w1[2], w1[3]);
    dst1[1] = make_uint4(w1[4], w1[5], w1[6], w1[7]);
  }
  for (int d = tid; d < K; d += kThreads) {
    const float e = __expf(Gc[(kL - 1) * GP + d]);
    p.egl[size_t(cid) * K + d] = e;
    if constexpr (BT) bt.egl[size_t(cid) * K + d] = e;
  }
  if constexpr (BT) {
    // Kc = e^{G_last−G}⊙K row-major (the same products as Kcᵀ).
#pragma unroll
    for (int m = 0; m < NLD; ++m) {
      const int idx = tid + kThreads * m, t = idx / KS8, d0 = 8 * (idx % KS8);
      float kf[8], gt[8], gl[8], c[8];
      f8(*reinterpret_cast<const uint4*>(&Ks[sw(t, d0)]), kf);
      *reinterpret_cast<float4*>(gt) = *reinterpret_cast<const float4*>(&Gc[t * GP + d0]);
      *reinterpret_cast<float4*>(gt + 4) = *reinterpret_cast<const float4*>(&Gc[t * GP + d0 + 4]);
      *reinterpret_cast<float4*>(gl) = *reinterpret_cast<const float4*>(&Gc[(kL - 1) * GP + d0]);
      *reinterpret_cast<float4*>(gl + 4) =
          *reinterpret_cast<const float4*>(&Gc[(kL - 1) * GP + d0 + 4]);
#pragma unroll
      for (int x = 0; x < 8; ++x) c[x] = kf[x] * __expf(gl[x] - gt[x]);
      *reinterpret_cast<uint4*>(bt.Kc + (size_t(cid) * kL + t) * K + d0) =
          make_uint4(pk_bf16(c[0], c[1]), pk_bf16(c[2], c[3]), pk_bf16(c[4], c[5]),
                     pk_bf16(c[6], c[7]));
    }
  }
  __syncthreads();  // G is dead: T and the merge scratch take its space

  diag_inverse(A, Tm, wave, lane);
  // Zero T above the block diagonal (the merges never write there).
  for (int idx = tid; idx < kL * kL; idx += kThreads) {
    const int i = idx / kL, j = idx % kL;
    if (j / 16 > i / 16) Tm[i][j] = 0.f;
  }
  __syncthreads();
  merge_T(A, Tm, Xs, wave, lane, [] { __syncthreads(); });
  {
    const int row = tid / 4, c0 = 16 * (tid % 4);
    const size_t off = size_t(cid) * kL * kL + row * kL + c0;
    uint32_t tv[8], tl[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      const float x0 = Tm[row][c0 + 2 * c], x1 = Tm[row][c0 + 2 * c + 1];
      tv[c] = pk_bf16(x0, x1);
      tl[c] = pk_bf16(x0 - lo_f(tv[c]), x1 - hi_f(tv[c]));
    }
    uint4* tdst = reinterpret_cast<uint4*>(p.T + off);
    uint4* ldst = reinterpret_cast<uint4*>(p.Tlo + off);
    tdst[0] = make_uint4(tv[0], tv[1], tv[2], tv[3]);
    tdst[1] = make_uint4(tv[4], tv[5], tv[6], tv[7]);
    ldst[0] = make_uint4(tl[0], tl[1], tl[2], tl[3]);
    ldst[1] = make_uint4(tl[4], tl[5], tl[6], tl[7]);
    if constexpr (BT) {
      // Tᵀ row `row` = T's column `row`.
#pragma unroll
      for (int c = 0; c < 8; ++c) {
        const float x0 = Tm[c0 + 2 * c][row], x1 = Tm[c0 + 2 * c + 1][row];
        tv[c] = pk_bf16(x0, x1);
        tl[c] = pk_bf16(x0 - lo_f(tv[c]), x1 - hi_f(tv[c]));
      }
      uint4* ttd = reinterpret_cast<uint4*>(bt.Tt + off);
      uint4* tld = reinterpret_cast<uint4*>(bt.Ttl + off);
      ttd[0] = make_uint4(tv[0], tv[1], tv[2], tv[3]);
      ttd[1] = make_uint4(tv[4], tv[5], tv[6], tv[7]);
      tld[0] = make_uint4(tl[0], tl[1], tl[2], tl[3]);
      tld[1] = make_uint4(tl[4], tl[5], tl[6], tl[7]);
    }
  }
}

// ---------------------------------------------------------------------------
// Segmented scan: the carry between segments
// ---------------------------------------------------------------------------
// Over a segment the chunk update S ← A_n·S + B_n composes to S_end =
// M·S_start + H (M = Π A_n, H the end state from S = 0), which the scan's
// seg = 1 mode produces for every segment at once. Here one workgroup of
// four waves per (b, h, 16 state columns) walks its segments in order:
// start(0) = S_in, start(s+1) = M_s·start(s) + H_s, written to seg_start for
// the seg = 2 scan. Wave w forms state rows 32w … 32w+31; the four waves
// exchange the state through LDS once per step, and each holds its rows of
// the next M and H in registers, loaded while the current step finishes.
// The fp32 products run as bf16 MFMAs of hi + lo parts (Mh·Sh + Mh·Sl +
// Ml·Sh, relative error about 2⁻¹⁶).
template <int K>
__global__ __launch_bounds__(256) void seg_carry_kernel(MfmaParams p) {
  static_assert(K == 128, "four waves of 32 state rows");
  constexpr int KK = K / 32;
  __shared__ float Ss[K][17];  // the state's 16 columns
  const int ncol = p.V / 16, P = p.seg_p;
  const int bh = blockIdx.x / ncol, ct = blockIdx.x % ncol;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, r16 = lane & 15, q4 = lane >> 4;
  const int col = 16 * ct + r16, row0 = 32 * wave;
  f32x4 S[2];  // rows row0 + 16j + 4q4 + r
  {
    const float* sin = p.s_in + size_t(bh) * K * p.V + col;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[j][r] = sin[size_t(row0 + 16 * j + 4 * q4 + r) * p.V];
  }
  // This wave's rows of M_s (channels 32kk + 4q4 + 0…3 and 32kk + 16 + 4q4 +
  // 0…3, the B fragment's order) and of H_s.
  float4 mA[2][KK][2];
  f32x4 hA[2];
  auto fetch = [&](int s) {
    const size_t seg = size_t(b * P + s) * p.H + h;
    const float* M = p.seg_m + seg * K * K;
    const float* Hs = p.seg_h + seg * K * p.V + col;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const float* mr = M + size_t(row0 + 16 * j + r16) * K + 32 * kk + 4 * q4;
        mA[j][kk][0] = *reinterpret_cast<const float4*>(mr);
        mA[j][kk][1] = *reinterpret_cast<const float4*>(mr + 16);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) hA[j][r] = Hs[size_t(row0 + 16 * j + 4 * q4 + r) * p.V];
    }
  };
  auto as8 = [](const uint4& x) { return __builtin_bit_cast(bf16x8, x); };
  if (P > 1) fetch(0);
  for (int s = 0; s < P; ++s) {
    float* st = p.seg_start + (size_t(b * P + s) * p.H + h) * K * p.V + col;
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        st[size_t(row0 + 16 * j + 4 * q4 + r) * p.V] = S[j][r];
        Ss[row0 + 16 * j + 4 * q4 + r][r16] = S[j][r];
      }
    if (s + 1 == P) break;
    __syncthreads();  // the whole state is in Ss
    f32x4 acc[2] = {hA[0], hA[1]};
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) {
      f32x4 s0, s1;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        s0[r] = Ss[32 * kk + 4 * q4 + r][r16];
        s1[r] = Ss[32 * kk + 16 + 4 * q4 + r][r16];
      }
      const uint4 sh = frag_hi(s0, s1);
      const uint4 sl = frag_lo(s0, s1, sh);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float4 a0 = mA[j][kk][0], a1 = mA[j][kk][1];
        const f32x4 m0 = {a0.x, a0.y, a0.z, a0.w}, m1 = {a1.x, a1.y, a1.z, a1.w};
        const uint4 mh = frag_hi(m0, m1);
        const uint4 ml = frag_lo(m0, m1, mh);
        acc[j] = mfma16(as8(mh), as8(sh), acc[j]);
        acc[j] = mfma16(as8(mh), as8(sl), acc[j]);
        acc[j] = mfma16(as8(ml), as8(sh), acc[j]);
      }
    }
    if (s + 2 < P) fetch(s + 1);
    __syncthreads();  // every wave has read Ss
    S[0] = acc[0];
    S[1] = acc[1];
  }
}

// ---------------------------------------------------------------------------
// Backward: the reverse scan carrying the state cotangent dS
// ---------------------------------------------------------------------------
// combined_backward.rs:240-319, the dS recurrence, walking the chunks in
// reverse: with dS the cotangent of the state leaving chunk n,
//   dV' = attnᵀ·dY + Kc·dS
//   Z   = Tᵀ·dV'
//   dS  ← e^{G_last}⊙dS + Qgᵀ·dY − Kgᵀ·Z        (Wᵀ·dV' = kgᵀ·(Tᵀ·dV'))
// and writes each chunk's leaving dS (fp32) for the chunk-local gradients.
// Same layout as the forward scan: one workgroup per (b, h, 16·W value
// columns), a wave owns 16 columns and all K state rows of dS in fp32 MFMA
// accumulators; the chunk's tiles (Kc, attnᵀ, Tᵀ hi/lo, Qgᵀ, Kgᵀ) are staged
// once in double-buffered LDS with the same k-permutation (head_k_dim 256:
// 120 KB a chunk, single-buffered between two barriers). dS is read as bf16
// hi + lo parts, dV' likewise for Tᵀ·dV'.
struct RevParams {
  int B, S, H, V, N;
  const void* dy;            // [B, S, H, V], bf16 or fp32
  const float* dstate_final;  // [B, H, K, V] or null (zeros)
  float* ds_after;            // [G][K][V]
  float* dstate;              // [B, H, K, V] cotangent of the initial state
  BwdTiles bt;
};

// G4: ds_after in row groups of four ([G][K/4][V][4], states_g4).
template <int K, class TG, int WAVES, bool G4 = false>
__global__ __launch_bounds__(64 * WAVES) void mfma_rev_scan_kernel(RevParams p) {
  constexpr int KK = K / 32;
  constexpr int RBK = K / 16;
  constexpr int NT = 64 * WAVES;
  constexpr int BW = 16 * WAVES;
  // Tiles: Kc [64][K]; attnᵀ, Tᵀ, Tᵀlo [64][64]; Qgᵀ, Kgᵀ [K][64].
  constexpr int oKc = 0, oAt = kL * K, oTt = oAt + kL * kL, oTtl = oTt + kL * kL,
                oQg = oTtl + kL * kL, oKg = oQg + K * kL, BUF = oKg + K * kL;
  constexpr int C16 = BUF / 8;
  static_assert(C16 % NT == 0, "staging assumes whole rounds");
  constexpr int NPF = C16 / NT;
  constexpr int NK = kL * K / 8;                   // 16-byte chunks of the K-wide tile
  constexpr int N64 = 3 * kL * kL / 8;             // of the three 64×64 tiles
  constexpr int NBUF = K > 128 ? 1 : 2;
  __shared__ __attribute__((aligned(16))) uint16_t tiles[NBUF][BUF];
  __shared__ float gch[NBUF][K];

  const int ntile = p.V / BW;
  const int BH = p.B * p.H;
  const int id = blockIdx.x;
  const int group = id / (8 * ntile), within = id % (8 * ntile);
  const int tile = within / 8, bh = group * 8 + within % 8;
  if (bh >= BH) return;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, q4 = lane >> 4, k8 = 8 * q4;
  const int jw = tile * BW + 16 * wave;
  const int jl = jw + r16;
  const size_t tokstride = size_t(p.H);
  const size_t bh_row0 = size_t(b) * p.S * p.H + h;
  auto chunk_of = [&](int n) { return (size_t(b) * p.N + n) * p.H + h; };

  // One test of dstate_final around all the loads (a test per element made
  // each load a branch of its own, waited for before the next).
  f32x4 dS[RBK];
  if (p.dstate_final) {
#pragma unroll
    for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        dS[rb][r] = p.dstate_final[(size_t(bh) * K + 16 * rb + 4 * q4 + r) * p.V + jl];
  } else {
#pragma unroll
    for (int rb = 0; rb < RBK; ++rb) dS[rb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  uint4 pf[NPF];
  float pch;
  auto ld16 = [](const uint16_t* base, uint32_t elems) {
    return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + 2u * elems);
  };
  auto fetch = [&](int n) {
    const size_t cid = chunk_of(n);
#pragma unroll
    for (int m = 0; m < NPF; ++m) {
      const int i0 = NT * m;
      if (i0 < NK) {
        pf[m] = ld16(p.bt.Kc + cid * kL * K + 8 * i0, 8u * tid);
      } else if (i0 < NK + N64) {
        const int ii0 = i0 - NK, which = ii0 / (kL * kL / 8);
        const uint16_t* base = which == 0 ? p.bt.AtT : which == 1 ? p.bt.Tt : p.bt.Ttl;
        pf[m] = ld16(base + cid * kL * kL + 8 * (ii0 - which * (kL * kL / 8)), 8u * tid);
      } else {
        const int ii0 = i0 - NK - N64, which = ii0 / (K * kL / 8);
        const uint16_t* base = which == 0 ? p.bt.QgT : p.bt.KgT;
        pf[m] = ld16(base + cid * K * kL + 8 * (ii0 - which * (K * kL / 8)), 8u * tid);
      }
    }
    pch = p.bt.egl[cid * K + (tid % K)];
  };
  constexpr int KC8 = K / 8, LC8 = kL / 8;
  const int rK = tid / KC8, cK = tid % KC8, r6 = tid / LC8, c6 = tid % LC8;
  auto addr_k = [&](int flip, int half) {
    const int pos = perm_pos(8 * cK + 4 * half);
    return rK * K + ((((pos >> 3) ^ (rK & 15) ^ flip) & (KC8 - 1)) << 3) + (pos & 7);
  };
  const int aK0 = K >= 128 ? addr_k(0, 0) : tile_at<K>(rK, perm_pos(8 * cK));
  const int aK1 = K >= 128 ? addr_k(0, 1) : tile_at<K>(rK, perm_pos(8 * cK + 4));
  const int aK0x = K >= 128 ? addr_k(8, 0) : aK0;
  const int aK1x = K >= 128 ? addr_k(8, 1) : aK1;
  const int a60 = tile_at<kL>(r6, perm_pos(8 * c6)), a61 = tile_at<kL>(r6, perm_pos(8 * c6 + 4));
  auto stage = [&](int buf) {
    uint16_t* tl = tiles[buf];
#pragma unroll
    for (int m = 0; m < NPF; ++m) {
      const int i0 = NT * m;
      int b0, b1;
      if (i0 < NK) {
        const int dr = i0 / KC8;
        const bool flip = K >= 128 && (dr & 8);
        b0 = oKc + dr * K + (flip ? aK0x : aK0);
        b1 = oKc + dr * K + (flip ? aK1x : aK1);
      } else if (i0 < NK + N64) {
        const int ii0 = i0 - NK, which = ii0 / (kL * kL / 8);
        const int dr = (ii0 - which * (kL * kL / 8)) / LC8;
        const int base = (which == 0 ? oAt : which == 1 ? oTt : oTtl) + dr * kL;
        b0 = base + a60;
        b1 = base + a61;
      } else {
        const int ii0 = i0 - NK - N64, which = ii0 / (K * kL / 8);
        const int dr = (ii0 - which * (K * kL / 8)) / LC8;
        const int base = (which == 0 ? oQg : oKg) + dr * kL;
        b0 = base + a60;
        b1 = base + a61;
      }
      *reinterpret_cast<uint2*>(&tl[b0]) = make_uint2(pf[m].x, pf[m].y);
      *reinterpret_cast<uint2*>(&tl[b1]) = make_uint2(pf[m].z, pf[m].w);
    }
    if (tid < K) gch[buf][tid] = pch;
  };
  // dY[t][jl] for the 16 tokens of this lane's two B fragments (k = token,
  // permuted: position 8q+e ↔ token 4q+e, 8q+4+e ↔ token 16+4q+e of each
  // 32-token step); zero past the sequence end.
  float dyR[2][8];
  auto load_dy = [&](int n) {
    const int rl = min(kL, p.S - n * kL);
    const size_t base = (bh_row0 + size_t(n) * kL * tokstride) * p.V + jl;
    const size_t stride = tokstride * p.V;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = 32 * kk + (e < 4 ? 4 * q4 + e : 16 + 4 * q4 + e - 4);
        const size_t at = base + size_t(min(t, rl - 1)) * stride;
        const float v = ld(static_cast<const TG*>(p.dy), at);
        dyR[kk][e] = t < rl ? v : 0.f;
      }
  };
  auto as8 = [](const uint4& x) { return __builtin_bit_cast(bf16x8, x); };

  fetch(p.N - 1);
  load_dy(p.N - 1);
  stage(0);
  __syncthreads();
  for (int it = 0; it < p.N; ++it) {
    const int n = p.N - 1 - it;
    const int cur = NBUF == 1 ? 0 : (it & 1);
    const int nn = n > 0 ? n - 1 : n;  // the first chunk prefetches itself again
    const uint16_t* tl = tiles[cur];
    if constexpr (G4) {
      float4* dst = reinterpret_cast<float4*>(p.ds_after + chunk_of(n) * K * p.V) + jl;
#pragma unroll
      for (int rb = 0; rb < RBK; ++rb)
        dst[size_t(4 * rb + q4) * p.V] = make_float4(dS[rb][0], dS[rb][1], dS[rb][2], dS[rb][3]);
    } else {
      float* dst = p.ds_after + chunk_of(n) * K * p.V + jl;
#pragma unroll
      for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) dst[size_t(16 * rb + 4 * q4 + r) * p.V] = dS[rb][r];
    }
    fetch(nn);
    uint4 dyf[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      dyf[kk] = make_uint4(pk_bf16(dyR[kk][0], dyR[kk][1]), pk_bf16(dyR[kk][2], dyR[kk][3]),
                           pk_bf16(dyR[kk][4], dyR[kk][5]), pk_bf16(dyR[kk][6], dyR[kk][7]));

    // Phase 1: dV' = attnᵀ·dY + Kc·dS in [token][column] orientation.
    // Two-wave workgroups (one wave per SIMD) split each k-step's dS
    // fragments under the previous step's MFMAs (the first under attnᵀ·dY),
    // one MFMA to three VALU instructions: config 5's reverse scan 1010 →
    // 893 µs. With two waves per SIMD the other wave covers the split, and
    // so interleaved the eight-wave scan measured slower (875 → 904 µs).
    constexpr bool kPipe = WAVES == 2;
    f32x4 dV[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) dV[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    if constexpr (kPipe) {
      uint4 sh = frag_hi(dS[0], dS[1]);
      uint4 sl = frag_lo(dS[0], dS[1], sh);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          dV[tb] = mfma16(ld8(&tl[oAt + tile_at<kL>(16 * tb + r16, 32 * kk + k8)]),
                          as8(dyf[kk]), dV[tb]);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
        __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
      }
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        uint4 shn = sh, sln = sl;
        if (kk + 1 < KK) {
          shn = frag_hi(dS[2 * kk + 2], dS[2 * kk + 3]);
          sln = frag_lo(dS[2 * kk + 2], dS[2 * kk + 3], shn);
        }
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          const bf16x8 kf = ld8(&tl[oKc + tile_at<K>(16 * tb + r16, 32 * kk + k8)]);
          dV[tb] = mfma16(kf, as8(sh), dV[tb]);
          dV[tb] = mfma16(kf, as8(sl), dV[tb]);
        }
        if (kk + 1 < KK) {
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
            __builtin_amdgcn_sched_group_barrier(0x002, 3, 0);  // three VALU
          }
        }
        sh = shn;
        sl = sln;
      }
    } else {
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          dV[tb] = mfma16(ld8(&tl[oAt + tile_at<kL>(16 * tb + r16, 32 * kk + k8)]),
                          as8(dyf[kk]), dV[tb]);
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) {
        const uint4 sh = frag_hi(dS[2 * kk], dS[2 * kk + 1]);
        const uint4 sl = frag_lo(dS[2 * kk], dS[2 * kk + 1], sh);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          const bf16x8 kf = ld8(&tl[oKc + tile_at<K>(16 * tb + r16, 32 * kk + k8)]);
          dV[tb] = mfma16(kf, as8(sh), dV[tb]);
          dV[tb] = mfma16(kf, as8(sl), dV[tb]);
        }
      }
    }
    load_dy(nn);

    // Phase 2: Z = Tᵀ·dV' with hi + lo parts of both factors.
    // (Tᵀ and attnᵀ are upper triangular, but skipping their zero blocks
    // here measured slower: 1010 → 1265 µs for the two-wave reverse scan of
    // BASELINE config 5, with the same register use.)
    uint4 vh[2], vl[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      vh[kk] = frag_hi(dV[2 * kk], dV[2 * kk + 1]);
      vl[kk] = frag_lo(dV[2 * kk], dV[2 * kk + 1], vh[kk]);
    }
    f32x4 Z[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      Z[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int at = tile_at<kL>(16 * tb + r16, 32 * kk + k8);
        const bf16x8 th = ld8(&tl[oTt + at]), tlo = ld8(&tl[oTtl + at]);
        Z[tb] = mfma16(th, as8(vh[kk]), Z[tb]);
        Z[tb] = mfma16(tlo, as8(vh[kk]), Z[tb]);
        Z[tb] = mfma16(th, as8(vl[kk]), Z[tb]);
      }
    }

    // Phase 3: dS ← e^{G_last}⊙dS + Qgᵀ·dY − Kgᵀ·Z.
    uint4 zf[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      f32x4 a = Z[2 * kk], c = Z[2 * kk + 1];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        a[r] = -a[r];
        c[r] = -c[r];
      }
      zf[kk] = frag_hi(a, c);
    }
#pragma unroll
    for (int rb = 0; rb < RBK; ++rb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) dS[rb][r] *= gch[cur][16 * rb + 4 * q4 + r];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const int at = tile_at<kL>(16 * rb + r16, 32 * kk + k8);
        dS[rb] = mfma16(ld8(&tl[oQg + at]), as8(dyf[kk]), dS[rb]);
        dS[rb] = mfma16(ld8(&tl[oKg + at]), as8(zf[kk]), dS[rb]);
      }
    }
    if constexpr (NBUF == 1) {
      __syncthreads();  // every wave is done with this chunk's tiles
      stage(0);
    } else {
      stage(cur ^ 1);
    }
    __syncthreads();
  }
  float* dout = p.dstate + size_t(bh) * K * p.V + jl;
#pragma unroll
  for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) dout[size_t(16 * rb + 4 * q4 + r) * p.V] = dS[rb][r];
}

size_t region(size_t bytes) { return align_up(bytes, 256); }

// Per-key-channel decay (GDN-2): the block-decay scores and the kg/qg tiles.
bool per_channel(const Dims& d) { return d.dw == d.K && d.K > 1; }
// The per-channel kernels: a per-key-channel forget gate, or a per-channel
// erase or write gate beside a per-head (or no) forget gate, which they serve
// with the head mask (mfma_intra_pc_kernel's HD).
bool pc_path(const Dims& d) { return per_channel(d) || d.ew > 1 || d.ww > 1; }

MfmaParams make_params(const Dims& d, const void* q, const void* k, const void* v,
                       const float* erase, const float* write, const float* g,
                       const float* state_in, void* y, float* state_out, void* ws) {
  const size_t G = size_t(d.B) * d.N * d.H;
  MfmaParams p;
  p.B = d.B;
  p.S = d.S;
  p.H = d.H;
  p.V = d.V;
  p.N = d.N;
  p.gated = d.dw > 0;
  p.scale = d.scale;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.erase = erase;
  p.write = write;
  p.g = g;
  p.s_in = state_in;
  p.y = y;
  p.s_out = state_out;
  p.ew = int(d.ew);
  p.ww = int(d.ww);
  p.states = nullptr;
  p.seg = 0;
  p.seg_p = 1;
  p.vx = d.V;
  p.seg_m = p.seg_h = p.seg_start = p.seg_final = nullptr;
  char* base = static_cast<char*>(ws);
  p.T = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * kL * 2);
  p.Tlo = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * kL * 2);
  p.attn = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * kL * 2);
  p.gc = reinterpret_cast<float*>(base);
  base += region(G * kL * 4);
  // Kcᵀ: per-channel gates only (with per-head gates the scan forms it from
  // the K tile).
  p.KcT = nullptr;
  if (pc_path(d)) {
    p.KcT = reinterpret_cast<uint16_t*>(base);
    base += region(G * size_t(d.K) * kL * 2);
  }
  p.sink = reinterpret_cast<uint16_t*>(base);
  base += region(size_t(d.V) * 4);
  p.Kg = p.Kglo = p.Qg = nullptr;
  p.egl = nullptr;
  if (pc_path(d)) {
    p.Kg = reinterpret_cast<uint16_t*>(base);
    base += region(G * kL * size_t(d.K) * 2);
    p.Kglo = reinterpret_cast<uint16_t*>(base);
    base += region(G * kL * size_t(d.K) * 2);
    p.Qg = reinterpret_cast<uint16_t*>(base);
    base += region(G * kL * size_t(d.K) * 2);
    p.egl = reinterpret_cast<float*>(base);
  }
  return p;
}

// The two-kernel forward's tiles (make_params' layout).
size_t tiles_workspace(const Dims& d) {
  const size_t G = size_t(d.B) * d.N * d.H;
  size_t bytes = 3 * region(G * kL * kL * 2) + region(G * kL * 4) + region(size_t(d.V) * 4);
  if (pc_path(d))
    bytes += region(G * size_t(d.K) * kL * 2) + 3 * region(G * kL * size_t(d.K) * 2) +
             region(G * size_t(d.K) * 4);
  return bytes;
}

// The backward's transposed tiles, after the forward's tiles.
BwdTiles carve_bwd_tiles(const Dims& d, void* ws) {
  const size_t G = size_t(d.B) * d.N * d.H, K = size_t(d.K);
  char* base = static_cast<char*>(ws) + tiles_workspace(d);
  BwdTiles bt;
  bt.Tt = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * kL * 2);
  bt.Ttl = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * kL * 2);
  bt.AtT = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * kL * 2);
  bt.Kc = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * K * 2);
  bt.QgT = reinterpret_cast<uint16_t*>(base);
  base += region(G * K * kL * 2);
  bt.KgT = reinterpret_cast<uint16_t*>(base);
  base += region(G * K * kL * 2);
  bt.egl = reinterpret_cast<float*>(base);
  return bt;
}

// bt (per-channel gates only): also write the backward's transposed tiles.
// Workgroups of `threads` threads of kernel `fn` resident on one CU at once
// (at least 1), cached per device and kernel.
int resident_per_cu(const void* fn, int threads) {
  static std::mutex mu;
  static std::map<std::pair<int, const void*>, int> cache;
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess) return 1;
  std::lock_guard<std::mutex> lock(mu);
  auto it = cache.find({dev, fn});
  if (it != cache.end()) return it->second;
  int n = 0;
  if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&n, fn, threads, 0) != hipSuccess || n < 1)
    n = 1;
  cache[{dev, fn}] = n;
  return n;
}

hipError_t launch_intra(const MfmaParams& p, const Dims& d, hipStream_t stream,
                        const BwdTiles* bt = nullptr, const FeParams* fe = nullptr) {
  const size_t G = size_t(d.B) * d.N * d.H;
  if (fe) {
    // The front-end's q/k in the load stage (per-head gates, head_k_dim 128):
    // a grid that is a multiple of nheads, so that each workgroup keeps one
    // head's conv weights.
    ProfScope ps("dn_mfma_intra_fe", stream);
    const void* fn = p.gated ? reinterpret_cast<const void*>(&mfma_intra_kernel<128, true, false, true>)
                             : reinterpret_cast<const void*>(&mfma_intra_kernel<128, false, false, true>);
    const size_t cap = size_t(resident_per_cu(fn, kThreads)) * device_cu_count();
    const size_t H = size_t(d.H);
    const size_t grid = std::max(H, std::min(G, cap) / H * H);
    if (p.gated)
      hipLaunchKernelGGL((mfma_intra_kernel<128, true, false, true>), dim3(unsigned(grid)),
                         dim3(kThreads), 0, stream, p, int(G), BwdTiles{}, *fe);
    else
      hipLaunchKernelGGL((mfma_intra_kernel<128, false, false, true>), dim3(unsigned(grid)),
                         dim3(kThreads), 0, stream, p, int(G), BwdTiles{}, *fe);
    return hipGetLastError();
  }
  if (pc_path(d)) {
    ProfScope ps(bt ? "dn_mfma_intra_pc_bwd" : "dn_mfma_intra_pc", stream);
    const bool hd = !per_channel(d);
#define DN_IPC(KD, BTV, EW)                                                                        \
  do {                                                                                           \
    if (hd)                                                                                      \
      hipLaunchKernelGGL((mfma_intra_pc_kernel<KD, BTV, EW, true>), dim3(unsigned(G)),           \
                         dim3(kThreads), 0, stream, p, bt ? *bt : BwdTiles{});                   \
    else                                                                                         \
      hipLaunchKernelGGL((mfma_intra_pc_kernel<KD, BTV, EW>), dim3(unsigned(G)), dim3(kThreads), \
                         0, stream, p, bt ? *bt : BwdTiles{});                                   \
  } while (0)
#define DN_IPC_E(KD, BTV)                         \
  do {                                            \
    if (d.ew == 1) DN_IPC(KD, BTV, true);         \
    else DN_IPC(KD, BTV, false);                  \
  } while (0)
    if (d.K == 128) {
      if (bt) DN_IPC_E(128, true); else DN_IPC_E(128, false);
    } else {
      if (bt) DN_IPC_E(64, true); else DN_IPC_E(64, false);
    }
#undef DN_IPC_E
#undef DN_IPC
  } else {
    // As many workgroups as are resident at once walk all chunk-heads: a
    // workgroup that had to wait for a slot would double the tail.
    ProfScope ps(bt ? "dn_mfma_intra_bwd" : "dn_mfma_intra", stream);
#define DN_INTRA(KD, GT, BTV)                                                                    \
  do {                                                                                           \
    const void* fn = reinterpret_cast<const void*>(&mfma_intra_kernel<KD, GT, BTV>);             \
    const int grid = int(std::min<size_t>(G, size_t(resident_per_cu(fn, kThreads)) *             \
                                                 device_cu_count()));                            \
    hipLaunchKernelGGL((mfma_intra_kernel<KD, GT, BTV>), dim3(unsigned(grid)), dim3(kThreads),   \
                       0, stream, p, int(G), bt ? *bt : BwdTiles{}, FeParams{});                 \
  } while (0)
#define DN_INTRA_G(KD, BTV)                              \
  do {                                                   \
    if (p.gated) DN_INTRA(KD, true, BTV);                \
    else DN_INTRA(KD, false, BTV);                       \
  } while (0)
    if (d.K == 256) {
      if (bt) DN_INTRA_G(256, true); else DN_INTRA_G(256, false);
    } else if (d.K == 128) {
      if (bt) DN_INTRA_G(128, true); else DN_INTRA_G(128, false);
    } else {
      if (bt) DN_INTRA_G(64, true); else DN_INTRA_G(64, false);
    }
#undef DN_INTRA_G
#undef DN_INTRA
  }
  return hipGetLastError();
}

// Scan workgroup width: 128 or 64 value columns (8 or 4 waves) when that
// still yields a workgroup per CU, else 32 so more CUs share the sequences
// (config 4, 64 sequences of dv = 128: 256 two-wave workgroups run its scan
// 3% faster than 128 four-wave ones).
int scan_waves(const Dims& d) {
  // head_k_dim 256: eight waves, whose staging registers (11 per lane) fit
  // beside the 64 of the state's rows.
  if (d.K == 256) return 8;
  const int groups = (d.B * d.H + 7) / 8;
  const int cus = device_cu_count();
  if (d.V % 128 == 0 && size_t(groups) * 8 * (d.V / 128) >= size_t(cus)) return 8;
  if (d.V % 64 == 0 && size_t(groups) * 8 * (d.V / 64) >= size_t(cus)) return 4;
  return 2;
}

// Segments per sequence for the scans. A scan workgroup holds a CU's LDS,
// and 8-wave workgroups do about twice the work per CU of the 2-wave ones
// the unsegmented scan falls back to, while segmenting triples the scans'
// work (the transitions cover K extra columns, then the outputs). So the
// sequence is cut only when even 2-wave workgroups would leave half the
// device idle, into enough segments to fill it with 8-wave workgroups, of
// at least 16 whole chunks each (head_k_dim 128, head_v_dim a multiple of
// 128, a sequence of whole chunks).
int seg_parts(const Dims& d) {
  if (d.K != 128 || d.V % 128 != 0 || size_t(d.S) != size_t(d.N) * d.L) return 1;
  const size_t cus = size_t(device_cu_count());
  if (size_t(d.B) * d.H * (d.V / 32) * 2 > cus) return 1;
  const size_t wgs = size_t(d.B) * d.H * (d.V / 128);
  int P = 1;
  while (wgs * P * 2 <= cus && d.N % (P * 2) == 0 && d.N / (P * 2) >= 16) P *= 2;
  return P;
}

// The segmented scan's buffers, after the tiles in the workspace.
size_t seg_workspace(const Dims& d) {
  const int P = seg_parts(d);
  if (P == 1) return 0;
  const size_t bh = size_t(d.B) * P * d.H, K = size_t(d.K);
  return region(bh * K * K * 4) + 2 * region(bh * K * d.V * 4);
}

void carve_seg(MfmaParams& p, const Dims& d, void* seg_ws) {
  const size_t bh = size_t(d.B) * seg_parts(d) * d.H, K = size_t(d.K);
  char* base = static_cast<char*>(seg_ws);
  p.seg_m = reinterpret_cast<float*>(base);
  base += region(bh * K * K * 4);
  p.seg_h = reinterpret_cast<float*>(base);
  base += region(bh * K * d.V * 4);
  p.seg_start = reinterpret_cast<float*>(base);
}

// The dims of the segmented scans: batch b·P + s runs segment s of batch b.
Dims seg_dims(const Dims& d, int P) {
  Dims s = d;
  s.B = d.B * P;
  s.S = d.S / P;
  s.N = d.N / P;
  return s;
}

// g4 (ST): write the states in row groups of four (states_g4).
template <bool ST>
hipError_t launch_scan(const MfmaParams& p, const Dims& d, bool yb, hipStream_t stream,
                       bool g4 = false) {
  const bool pc = pc_path(d);
  if constexpr (!ST) {
    if (p.seg) {
      // The segmented scans: 8-wave workgroups, head_k_dim 128.
      const unsigned blocks = unsigned(((d.B * d.H + 7) / 8) * 8 * (p.vx / 128));
      ProfScope ps(p.seg == 1 ? (pc ? "dn_mfma_scan_pc_segs" : "dn_mfma_scan_segs")
                              : (pc ? "dn_mfma_scan_pc" : "dn_mfma_scan"),
                   stream);
#define DN_SEG(TY, SG)                                                                           \
  do {                                                                                           \
    if (pc)                                                                                      \
      hipLaunchKernelGGL((mfma_scan_kernel<128, TY, 8, true, false, SG>), dim3(blocks),          \
                         dim3(512), 0, stream, p);                                               \
    else                                                                                         \
      hipLaunchKernelGGL((mfma_scan_kernel<128, TY, 8, false, false, SG>), dim3(blocks),         \
                         dim3(512), 0, stream, p);                                               \
  } while (0)
      if (p.seg == 1)
        DN_SEG(float, 1);  // no y
      else if (yb)
        DN_SEG(bf16, 2);
      else
        DN_SEG(float, 2);
#undef DN_SEG
      return hipGetLastError();
    }
  }
  const int waves = scan_waves(d);
  const unsigned blocks = unsigned(((d.B * d.H + 7) / 8) * 8 * (d.V / (16 * waves)));
  ProfScope ps(ST ? (pc ? "dn_mfma_scan_pc_states" : "dn_mfma_scan_states")
                  : (pc ? "dn_mfma_scan_pc" : "dn_mfma_scan"),
               stream);
#define DN_SCAN(KD, TY, W)                                                                        \
  do {                                                                                            \
    if (pc)                                                                                       \
      hipLaunchKernelGGL((mfma_scan_kernel<KD, TY, W, true, ST>), dim3(blocks), dim3(64 * W), 0,  \
                         stream, p);                                                              \
    else                                                                                          \
      hipLaunchKernelGGL((mfma_scan_kernel<KD, TY, W, false, ST>), dim3(blocks), dim3(64 * W), 0, \
                         stream, p);                                                              \
  } while (0)
#define DN_SCAN_W(KD, TY) \
  do { if (waves == 8) DN_SCAN(KD, TY, 8); else if (waves == 4) DN_SCAN(KD, TY, 4); else DN_SCAN(KD, TY, 2); } while (0)
  if constexpr (ST) {
    if (g4) {
      // Eight-wave workgroups (head_k_dim 64, 128, 256).
      if (waves != 8 || (pc && d.K == 256)) return hipErrorInvalidValue;
#define DN_SCAN_G4(KD, PCV)                                                                    \
  hipLaunchKernelGGL((mfma_scan_kernel<KD, float, 8, PCV, true, 0, 0, true>), dim3(blocks),     \
                     dim3(512), 0, stream, p)
      if (d.K == 256) DN_SCAN_G4(256, false);
      else if (d.K == 128) { if (pc) DN_SCAN_G4(128, true); else DN_SCAN_G4(128, false); }
      else { if (pc) DN_SCAN_G4(64, true); else DN_SCAN_G4(64, false); }
#undef DN_SCAN_G4
      return hipGetLastError();
    }
  }
  if (d.K == 256) {
    // head_k_dim 256: per-head gates, eight-wave workgroups.
    if (pc || waves != 8) return hipErrorInvalidValue;
    if constexpr (ST) {
      hipLaunchKernelGGL((mfma_scan_kernel<256, float, 8, false, true>), dim3(blocks), dim3(512),
                         0, stream, p);
    } else {
      if (yb)
        hipLaunchKernelGGL((mfma_scan_kernel<256, bf16, 8, false>), dim3(blocks), dim3(512), 0,
                           stream, p);
      else
        hipLaunchKernelGGL((mfma_scan_kernel<256, float, 8, false>), dim3(blocks), dim3(512), 0,
                           stream, p);
    }
  } else if (d.K == 128) {
    if (yb && !ST) DN_SCAN_W(128, bf16); else DN_SCAN_W(128, float);
  } else {
    if (yb && !ST) DN_SCAN_W(64, bf16); else DN_SCAN_W(64, float);
  }
#undef DN_SCAN_W
#undef DN_SCAN
  return hipGetLastError();
}

// Clears the output norm's exchange words (a fill kernel: the launch may be
// captured into a HIP graph, where memset nodes are avoided).
__global__ __launch_bounds__(256) void zero_words_kernel(unsigned long long* w, size_t n) {
  for (size_t i = size_t(blockIdx.x) * 256 + threadIdx.x; i < n; i += size_t(gridDim.x) * 256)
    w[i] = 0ull;
}

// The exchange words of the output norm: [B·P·H][V/32][4][64] (room for the
// narrowest scan workgroups), and the words a launch of `waves`-wave
// workgroups uses.
size_t norm_words(const Dims& d, int P, int waves) {
  return size_t(d.B) * P * d.H * (d.V / (16 * waves)) * 4 * kL;
}
size_t norm_exchange_bytes(const Dims& d) { return region(norm_words(d, seg_parts(d), 2) * 8); }

// The output-norm scan's launch geometry for dims `d` (the segmented output
// pass's dims when seg): workgroup waves and column workgroups per head.
struct NormLaunch {
  const void* fn;
  int waves, ntile;
  unsigned blocks;
};
NormLaunch norm_launch(const Dims& d, bool seg, bool yb, bool gated) {
  NormLaunch l;
  l.waves = seg ? 8 : scan_waves(d);
  l.ntile = d.V / (16 * l.waves);
  l.blocks = unsigned(((d.B * d.H + 7) / 8) * 8 * l.ntile);
  l.fn = norm_scan_fn(d.K, pc_path(d), seg, yb, l.waves, gated);
  return l;
}

// When a head's columns span several workgroups, they exchange per-token
// sums mid-kernel, so the whole grid must be resident: a cooperative launch.
// hipErrorCooperativeLaunchTooLarge when the device cannot hold it (the
// caller then runs the plain forward and a separate norm pass).
hipError_t norm_launch_fits(const NormLaunch& l) {
  if (l.ntile == 1) return hipSuccess;
  int per_cu = 0;
  hipError_t e = hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, l.fn, 64 * l.waves, 0);
  if (e != hipSuccess) return e;
  return size_t(per_cu) * device_cu_count() >= l.blocks ? hipSuccess
                                                         : hipErrorCooperativeLaunchTooLarge;
}

hipError_t launch_scan_norm(const MfmaParams& p, const Dims& d, bool yb, hipStream_t stream) {
  const NormLaunch l = norm_launch(d, p.seg != 0, yb, p.ng != nullptr);
  MfmaParams q = p;
  {
    const size_t nw = norm_words(d, 1, l.waves);
    hipLaunchKernelGGL(zero_words_kernel, dim3(unsigned(std::min<size_t>((nw + 255) / 256, 1024))),
                       dim3(256), 0, stream, q.nx, nw);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  ProfScope ps(pc_path(d) ? "dn_mfma_scan_pc_norm" : "dn_mfma_scan_norm", stream);
  void* args[] = {&q};
  if (l.ntile == 1) return hipLaunchKernel(l.fn, dim3(l.blocks), dim3(64 * l.waves), args, 0, stream);
  return hipLaunchCooperativeKernel(l.fn, dim3(l.blocks), dim3(64 * l.waves), args, 0, stream);
}

}  // namespace

bool mfma_fwd_supported(const Dims& d, int qkv_dtype, int y_dtype) {
  (void)y_dtype;
  if (!(qkv_dtype == DN_BF16 && d.V % kBV == 0 && d.L == kL)) return false;
  if (!token_rows_fit_32bit(d)) return false;
  // head_k_dim 256: per-head (or no) gates, eight-wave scan workgroups of
  // 128 value columns.
  if (d.K == 256) return !pc_path(d) && d.ew == 1 && d.ww == 1 && d.dw <= 1 && d.V % 128 == 0;
  if (d.K != 64 && d.K != 128) return false;
  if (pc_path(d)) return (d.ew == 1 || d.ew == d.K) && (d.ww == 1 || d.ww == d.V);
  return d.ew == 1 && d.ww == 1 && d.dw <= 1;
}

// The MFMA backward: its chunk-local kernel and scans know the per-head
// gates and the all-per-channel ones (GDN-2), at head_k_dim 64 and 128, and
// the per-head gates at head_k_dim 256; per-channel erase or write gates
// beside a per-head forget gate take the generic kernels.
bool mfma_bwd_supported(const Dims& d, int qkv_dtype) {
  if (!mfma_fwd_supported(d, qkv_dtype, DN_BF16)) return false;
  // head_k_dim 256: per-head gates (the forward's condition), width-1 gates
  if (d.K == 256) return true;
  return d.K <= 128 && (per_channel(d) || (d.ew == 1 && d.ww == 1));
}

size_t mfma_fwd_workspace(const Dims& d, bool fused) {
  return fused ? fused_fwd_workspace(d) : tiles_workspace(d) + seg_workspace(d);
}

hipError_t mfma_fwd(const Dims& d, int y_dtype, const void* q, const void* k, const void* v,
                    const float* erase, const float* write, const float* g,
                    const float* state_in, void* y, float* state_out, void* ws,
                    hipStream_t stream, bool fused, const FeParams* fe) {
  if (fused)
    return fused_fwd(d, y_dtype, q, k, v, erase, write, g, state_in, y, state_out, ws, stream);
  MfmaParams p = make_params(d, q, k, v, erase, write, g, state_in, y, state_out, ws);
  hipError_t e = launch_intra(p, d, stream, nullptr, fe);
  if (e != hipSuccess) return e;
  const int P = seg_parts(d);
  if (P == 1) return launch_scan<false>(p, d, y_dtype == DN_BF16, stream);
  // Segmented: the segments' transitions, the carry, then the outputs.
  carve_seg(p, d, static_cast<char*>(ws) + tiles_workspace(d));
  const Dims ds = seg_dims(d, P);
  MfmaParams pa = p;
  pa.B = ds.B;
  pa.S = ds.S;
  pa.N = ds.N;
  pa.seg = 1;
  pa.seg_p = P;
  pa.vx = d.V + d.K;
  pa.y = nullptr;
  if ((e = launch_scan<false>(pa, ds, y_dtype == DN_BF16, stream)) != hipSuccess) return e;
  {
    ProfScope ps("dn_mfma_seg_carry", stream);
    MfmaParams pb = p;
    pb.seg_p = P;
    hipLaunchKernelGGL(seg_carry_kernel<128>, dim3(unsigned(d.B * d.H * (d.V / 16))), dim3(256),
                       0, stream, pb);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  MfmaParams pc = pa;
  pc.seg = 2;
  pc.vx = d.V;
  pc.s_in = p.seg_start;
  pc.y = y;
  pc.seg_final = state_out;
  return launch_scan<false>(pc, ds, y_dtype == DN_BF16, stream);
}

size_t mfma_fwd_norm_workspace(const Dims& d) {
  return tiles_workspace(d) + seg_workspace(d) + norm_exchange_bytes(d);
}

hipError_t mfma_fwd_norm(const Dims& d, int y_dtype, const void* q, const void* k, const void* v,
                         const float* erase, const float* write, const float* g,
                         const float* state_in, void* y, float* state_out, void* ws,
                         const FwdNorm& nm, hipStream_t stream) {
  MfmaParams p = make_params(d, q, k, v, erase, write, g, state_in, y, state_out, ws);
  p.ng = nm.gate;
  p.ng_stride = nm.gate_stride;
  p.nw = nm.weight;
  p.neps = nm.eps;
  p.nx = reinterpret_cast<unsigned long long*>(static_cast<char*>(ws) + tiles_workspace(d) +
                                               seg_workspace(d));
  p.nfault = nm.fault;
  p.nspin = nm.spin;
  const int P = seg_parts(d);
  // Whether the scan can run as launched, decided before any launch so that
  // the caller's fallback starts from a clean slate.
  {
    hipError_t e = norm_launch_fits(norm_launch(P > 1 ? seg_dims(d, P) : d, P > 1,
                                                y_dtype == DN_BF16, nm.gate != nullptr));
    if (e != hipSuccess) return e;
  }
  hipError_t e = launch_intra(p, d, stream);
  if (e != hipSuccess) return e;
  if (P == 1) return launch_scan_norm(p, d, y_dtype == DN_BF16, stream);
  carve_seg(p, d, static_cast<char*>(ws) + tiles_workspace(d));
  const Dims ds = seg_dims(d, P);
  MfmaParams pa = p;
  pa.B = ds.B;
  pa.S = ds.S;
  pa.N = ds.N;
  pa.seg = 1;
  pa.seg_p = P;
  pa.vx = d.V + d.K;
  pa.y = nullptr;
  if ((e = launch_scan<false>(pa, ds, y_dtype == DN_BF16, stream)) != hipSuccess) return e;
  {
    ProfScope ps("dn_mfma_seg_carry", stream);
    MfmaParams pb = p;
    pb.seg_p = P;
    hipLaunchKernelGGL(seg_carry_kernel<128>, dim3(unsigned(d.B * d.H * (d.V / 16))), dim3(256),
                       0, stream, pb);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  MfmaParams pc = pa;
  pc.seg = 2;
  pc.vx = d.V;
  pc.s_in = p.seg_start;
  pc.y = y;
  pc.seg_final = state_out;
  return launch_scan_norm(pc, ds, y_dtype == DN_BF16, stream);
}

MfmaTiles mfma_bwd_tiles(const Dims& d, void* ws) {
  const MfmaParams p =
      make_params(d, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr, ws);
  const BwdTiles bt = carve_bwd_tiles(d, ws);
  return MfmaTiles{p.T, p.Tlo, bt.Tt, bt.Ttl, bt.AtT, bt.Kc, p.Kg, p.Kglo, p.gc};
}

size_t mfma_bwd_workspace(const Dims& d) {
  const size_t G = size_t(d.B) * d.N * d.H, K = size_t(d.K);
  return tiles_workspace(d) + 3 * region(G * kL * kL * 2) + region(G * kL * K * 2) +
         2 * region(G * K * kL * 2) + region(G * K * 4) +
         region(size_t(d.B) * d.H * K * d.V * 4);  // the recompute's final state (unused)
}

bool states_g4(const Dims& d) { return d.K == 256; }

hipError_t mfma_bwd_scans(const Dims& d, int grad_dtype, const void* dy,
                          const float* dstate_final, const void* q, const void* k, const void* v,
                          const float* erase, const float* write, const float* g,
                          const float* state_in, float* states, float* ds_after, float* dstate,
                          void* ws, hipStream_t stream, bool g4) {
  const size_t G = size_t(d.B) * d.N * d.H, K = size_t(d.K);
  // The forward recompute (states mode) and the reverse scan need nothing
  // from each other: after the intra kernel, the reverse scan and its tiles
  // run on the device's second stream, overlapping the recompute (each scan
  // alone fills few CUs when batch × heads is small). The recompute's final
  // state goes to a scratch region of the workspace.
  const BwdTiles bt = carve_bwd_tiles(d, ws);
  float* s_scratch = reinterpret_cast<float*>(reinterpret_cast<char*>(bt.egl) + region(G * K * 4));
  MfmaParams p = make_params(d, q, k, v, erase, write, g, state_in, nullptr, s_scratch, ws);
  p.states = states;
  // The states mode reads neither attn nor qg (the intra kernels form attn for
  // attnᵀ and write neither).
  p.attn = nullptr;
  // The intra kernel writes the reverse scan's transposed tiles too.
  hipError_t e = launch_intra(p, d, stream, &bt);
  if (e != hipSuccess) return e;
  hipStream_t side = nullptr;
  if ((e = side_fork(stream, &side)) != hipSuccess) return e;
  RevParams rp{d.B, d.S, d.H, d.V, d.N, dy, dstate_final, ds_after, dstate, bt};
  // head_k_dim 256: eight waves with ds_after in row groups of four (the
  // generic kernels' row-major layout: four, whose single wave per SIMD has
  // the register file for 256 dS rows beside the next chunk's 120 KB of
  // tiles; eight waves spilled there). At B=8 T=4096 H=16 dv=256: eight
  // waves row-major 5.05 ms, four 3.85, four in row groups 1.61, eight in
  // row groups 1.36.
  const int waves = d.K == 256 && !g4 ? 4 : scan_waves(d);
  const unsigned blocks = unsigned(((d.B * d.H + 7) / 8) * 8 * (d.V / (16 * waves)));
  {
  ProfScope ps("dn_mfma_rev_scan", side);
#define DN_REV(KD, TG, W) \
  hipLaunchKernelGGL((mfma_rev_scan_kernel<KD, TG, W>), dim3(blocks), dim3(64 * W), 0, side, rp)
#define DN_REV4(KD, TG, W)                                                                     \
  hipLaunchKernelGGL((mfma_rev_scan_kernel<KD, TG, W, true>), dim3(blocks), dim3(64 * W), 0,  \
                     side, rp)
#define DN_REV_W(KD, TG) \
  do { if (waves == 8) DN_REV(KD, TG, 8); else if (waves == 4) DN_REV(KD, TG, 4); else DN_REV(KD, TG, 2); } while (0)
  if (g4 && waves != 8 && d.K != 256) return hipErrorInvalidValue;
  if (d.K == 256) {
    if (g4) {
      if (grad_dtype == DN_BF16) DN_REV4(256, bf16, 8); else DN_REV4(256, float, 8);
    } else {
      if (grad_dtype == DN_BF16) DN_REV(256, bf16, 4); else DN_REV(256, float, 4);
    }
  } else if (g4) {
    if (d.K == 128) {
      if (grad_dtype == DN_BF16) DN_REV4(128, bf16, 8); else DN_REV4(128, float, 8);
    } else {
      if (grad_dtype == DN_BF16) DN_REV4(64, bf16, 8); else DN_REV4(64, float, 8);
    }
  } else if (d.K == 128) {
    if (grad_dtype == DN_BF16) DN_REV_W(128, bf16); else DN_REV_W(128, float);
  } else {
    if (grad_dtype == DN_BF16) DN_REV_W(64, bf16); else DN_REV_W(64, float);
  }
#undef DN_REV_W
#undef DN_REV4
#undef DN_REV
  }
  if ((e = hipGetLastError()) != hipSuccess) return e;
  if ((e = launch_scan<true>(p, d, false, stream, g4)) != hipSuccess) return e;
  return side_join(stream);
}

}  // namespace dn
