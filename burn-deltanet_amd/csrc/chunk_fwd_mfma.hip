// The chunkwise WY forward on CDNA4 matrix cores (bf16 MFMA, fp32 state).
//
// Covers the per-head gate shapes of Gated DeltaNet / DeltaNet / DeltaProduct:
// bf16 q/k/v, head_k_dim ∈ {64, 128}, head_v_dim a multiple of 64,
// chunk_len 64, erase/write/forget gates of width 1 (or no forget gate).
// Everything else takes the generic kernels.
//
// Two kernels, both on v_mfma_f32_16x16x32_bf16 (64-lane waves):
//
// intra  one workgroup per chunk-head (b, n, h); fully parallel.
//        K and Q chunk tiles are staged in LDS; K·Kᵀ and Q·Kᵀ (lower block
//        triangle only) run on MFMA; the per-head decay e^{Gᵢ−Gⱼ}, the erase
//        gate and the readout scale are applied to the fp32 accumulators;
//        T = (I + tril(Akk, −1))⁻¹ is a blocked forward substitution in fp32
//        LDS (four 16×16 diagonal inverses, then two doubling merges
//        T₂₁ = −T₂₂ A₂₁ T₁₁) — the reference's ladder (tri/prim.rs:28-51) at
//        L³/3 instead of 24·L³ flops. Writes T as bf16 hi + lo parts,
//        attn = tril(Aqk) as bf16 and the in-chunk cumulative gate G as fp32:
//        24.25 KiB per chunk-head.
//
// scan   one workgroup per (64-column value tile, head, batch); serial over
//        chunks. The fp32 state tile S [K × 64] lives in MFMA accumulator
//        registers for the whole sequence; a bf16 copy in LDS feeds the
//        products that read it. Per chunk, with U − W S = T (w⊙V − e⊙e^G⊙(K S))
//        so that neither U nor W is ever formed:
//          X  = w⊙V − (e⊙e^G)⊙(K·S)                 MFMA, K rows from HBM/L2;
//                                                   S read as bf16 hi + lo parts
//                                                   (the retrieval cancels)
//          V' = T·X                                 MFMA, hi + lo parts of T and X
//          y  = (scale·e^G)⊙(Q·S) + attn·V'         MFMA, written as bf16
//          S  ← e^{G_last}⊙S + (e^{G_last−G}⊙K)ᵀ·V' MFMA into the accumulators
//        The four tiles of one (b, h) are mapped to one XCD so their shared
//        K/Q/T/attn reads hit the same L2.

#include <algorithm>

#include "dn_common.hpp"

namespace dn {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int kL = 64;        // chunk length
constexpr int kThreads = 256;  // 4 waves
constexpr int kBV = 64;       // value columns per scan workgroup
constexpr int kZeroElems = 512;

__device__ inline f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;

__device__ inline bf16x8 ld8(const uint16_t* p) { return *reinterpret_cast<const bf16x8*>(p); }

// Two floats → packed bf16 (round to nearest even), one v_cvt_pk_bf16_f32.
__device__ inline uint32_t pk_bf16(float a, float b) {
  const bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
__device__ inline float lo_f(uint32_t u) { return __uint_as_float(u << 16); }
__device__ inline float hi_f(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

__device__ inline f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Value of lane `src` of each group of four lanes, to the whole group (DPP
// quad_perm); `src` folds to a constant once the caller's loop is unrolled.
template <int SRC>
__device__ inline float quad_bcast_c(float v) {
  return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v),
                                                 SRC | (SRC << 2) | (SRC << 4) | (SRC << 6),
                                                 0xf, 0xf, false));
}
__device__ inline float quad_bcast(float v, int src) {
  switch (src) {
    case 0: return quad_bcast_c<0>(v);
    case 1: return quad_bcast_c<1>(v);
    case 2: return quad_bcast_c<2>(v);
    default: return quad_bcast_c<3>(v);
  }
}

__device__ inline bf16x8 zero8() { return __builtin_bit_cast(bf16x8, make_uint4(0u, 0u, 0u, 0u)); }

struct MfmaParams {
  int B, S, H, V, N;
  int gated;
  float scale;
  const uint16_t *q, *k, *v;
  const float *erase, *write, *g;
  const float* s_in;
  void* y;
  float* s_out;
  uint16_t* T;     // [G][64][64] bf16(T)
  uint16_t* Tlo;   // [G][64][64] bf16(T − bf16(T))
  uint16_t* attn;  // [G][64][64] bf16
  uint16_t* KcT;   // [G][K][64] bf16 (e^{G_last−G}⊙K)ᵀ
  uint16_t* zero;  // kZeroElems bf16 zeros: the source of padded tokens' reads
  uint16_t* sink;  // one y row: the target of padded tokens' writes
  float* gc;       // [G][64]
};

// ---------------------------------------------------------------------------
// intra
// ---------------------------------------------------------------------------
template <int K, bool GATED>
__global__ __launch_bounds__(kThreads) void mfma_intra_kernel(MfmaParams p, int G) {
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

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  if (blockIdx.x == 0)
    for (int i = tid; i < kZeroElems / 8; i += kThreads)
      reinterpret_cast<uint4*>(p.zero)[i] = make_uint4(0u, 0u, 0u, 0u);
  // attn's blocks above the diagonal are zero for every chunk.
  for (int idx = tid; idx < kL * kL; idx += kThreads) {
    const int i = idx / kL, j = idx % kL;
    if (j / 16 > i / 16) At[i * (kL + 8) + j] = 0;
  }

  // The workgroup walks chunk-heads cid = blockIdx.x, + gridDim.x, …; the
  // next chunk's K, Q and gates are loaded into registers while this one
  // is processed.
  uint4 kr[NLD], qr[NLD];
  float gr = 0.f, er = 0.f;
  auto load = [&](int cid) {
    const int h = cid % p.H, n = (cid / p.H) % p.N, b = cid / (p.H * p.N);
#pragma unroll
    for (int m = 0; m < NLD; ++m) {
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
  if (int(blockIdx.x) < G) load(blockIdx.x);

  // T (hi, lo) and attn of the previous chunk, 16 values of one row per lane:
  // their global stores are issued after the next chunk is staged, so no
  // wait on them lands at the top of the loop.
  uint4 pend[6];
  int pend_cid = -1;
  auto store_pending = [&]() {
    const int row = tid / 4, c0 = 16 * (tid % 4);
    const size_t off = size_t(pend_cid) * kL * kL + row * kL + c0;
    uint4* tdst = reinterpret_cast<uint4*>(p.T + off);
    uint4* ldst = reinterpret_cast<uint4*>(p.Tlo + off);
    uint4* adst = reinterpret_cast<uint4*>(p.attn + off);
    tdst[0] = pend[0];
    tdst[1] = pend[1];
    ldst[0] = pend[2];
    ldst[1] = pend[3];
    adst[0] = pend[4];
    adst[1] = pend[5];
  };

  for (int cid = blockIdx.x; cid < G; cid += gridDim.x) {
#pragma unroll
    for (int m = 0; m < NLD; ++m) {
      const int idx = tid + kThreads * m, row = idx / KS8, c8 = idx % KS8;
      *reinterpret_cast<uint4*>(&Ks[row * KP + 8 * c8]) = kr[m];
      *reinterpret_cast<uint4*>(&Qs[row * KP + 8 * c8]) = qr[m];
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
    __syncthreads();

    {
      // T's diagonal 16×16 block `wave` by column elimination: lane (c, g)
      // holds rows g, g+4, g+8, g+12 of column c; step k₂ broadcasts x[k₂]
      // inside the lane quad (DPP) and updates the rows below it.
      const int base = 16 * wave, c = lane >> 2, g = lane & 3;
      float x[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) x[j] = (4 * j + g == c) ? 1.f : 0.f;
      // Multipliers A[i][k₂] for i > k₂ (zero otherwise), read up front.
      float mul[15][4];
#pragma unroll
      for (int k2 = 0; k2 < 15; ++k2)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int i = 4 * j + g;
          mul[k2][j] = (4 * j + 3 > k2 && i > k2) ? A[base + i][base + k2] : 0.f;
        }
#pragma unroll
      for (int k2 = 0; k2 < 15; ++k2) {
        const float xk = quad_bcast(x[k2 >> 2], k2 & 3);
#pragma unroll
        for (int j = 0; j < 4; ++j)
          if (4 * j + 3 > k2) x[j] -= mul[k2][j] * xk;
      }
#pragma unroll
      for (int j = 0; j < 4; ++j) Tm[base + 4 * j + g][base + c] = x[j];
    }
    {
      // Kcᵀ = (e^{G_last−G} ⊙ K)ᵀ for the scan's state update, while the K
      // tile is in LDS: an item is one key channel × 16 tokens, consecutive
      // lanes taking consecutive channels (conflict-free column reads).
      const float glast = gcs[kL - 1];
      for (int it = tid; it < K * 2; it += kThreads) {
        // Channels d, d+1 of 16 tokens: one 32-bit LDS read per token.
        const int d = 2 * (it % (K / 2)), t0 = 16 * (it / (K / 2));
        uint32_t w0[8], w1[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const int t = t0 + 2 * e;
          const uint32_t a = *reinterpret_cast<const uint32_t*>(&Ks[t * KP + d]);
          const uint32_t b = *reinterpret_cast<const uint32_t*>(&Ks[(t + 1) * KP + d]);
          const float s0 = GATED ? __expf(glast - gcs[t]) : 1.f;
          const float s1 = GATED ? __expf(glast - gcs[t + 1]) : 1.f;
          w0[e] = pk_bf16(lo_f(a) * s0, lo_f(b) * s1);
          w1[e] = pk_bf16(hi_f(a) * s0, hi_f(b) * s1);
        }
        uint4* dst0 = reinterpret_cast<uint4*>(p.KcT + (size_t(cid) * K + d) * kL + t0);
        uint4* dst1 = reinterpret_cast<uint4*>(p.KcT + (size_t(cid) * K + d + 1) * kL + t0);
        dst0[0] = make_uint4(w0[0], w0[1], w0[2], w0[3]);
        dst0[1] = make_uint4(w0[4], w0[5], w0[6], w0[7]);
        dst1[0] = make_uint4(w1[0], w1[1], w1[2], w1[3]);
        dst1[1] = make_uint4(w1[4], w1[5], w1[6], w1[7]);
      }
      // Zero T above the block diagonal (the merges never write there).
      for (int idx = tid; idx < kL * kL; idx += kThreads) {
        const int i = idx / kL, j = idx % kL;
        if (j / 16 > i / 16) Tm[i][j] = 0.f;
      }
    }
    __syncthreads();
    // The merges run on fp32 MFMA (v_mfma_f32_16x16x4_f32: exact fp32
    // products): lane l holds A[l%16][l/16] and B[l/16][l%16] of a
    // 16×4 · 4×16 step, and D[4(l/16)+r][l%16]. Full-block sums are exact:
    // the triangular factors hold zeros outside their triangles.
    const int m16 = lane & 15, g4 = lane >> 4;
    // 16 → 32: T₁₀ = −T₁₁ A₁₀ T₀₀ for the two 32-blocks (waves 0 and 1).
    if (wave < 2) {
      const int r0 = 32 * wave + 16, c0 = 32 * wave;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        acc = mfma_f32(A[r0 + m16][c0 + 4 * s4 + g4], Tm[c0 + 4 * s4 + g4][c0 + m16], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) Xs[16 * wave + 4 * g4 + r][m16] = acc[r];
    }
    __syncthreads();
    if (wave < 2) {
      const int r0 = 32 * wave + 16, c0 = 32 * wave;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        acc = mfma_f32(Tm[r0 + m16][r0 + 4 * s4 + g4], Xs[16 * wave + 4 * s4 + g4][m16], acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) Tm[r0 + 4 * g4 + r][c0 + m16] = -acc[r];
    }
    __syncthreads();
    // 32 → 64: T[32:,:32] = −T[32:,32:] A[32:,:32] T[:32,:32]; wave w owns
    // output tile (w/2, w%2) of the 32×32 block.
    {
      const int ti = wave >> 1, tj = wave & 1;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 8; ++s4)
        acc = mfma_f32(A[32 + 16 * ti + m16][4 * s4 + g4], Tm[4 * s4 + g4][16 * tj + m16], acc);
      __syncthreads();
#pragma unroll
      for (int r = 0; r < 4; ++r) Xs[16 * ti + 4 * g4 + r][16 * tj + m16] = acc[r];
      __syncthreads();
      acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s4 = 0; s4 < 8; ++s4)
        acc = mfma_f32(Tm[32 + 16 * ti + m16][32 + 4 * s4 + g4], Xs[4 * s4 + g4][16 * tj + m16],
                       acc);
#pragma unroll
      for (int r = 0; r < 4; ++r) Tm[32 + 16 * ti + 4 * g4 + r][16 * tj + m16] = -acc[r];
    }
    __syncthreads();

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
    }
    __syncthreads();  // LDS is restaged by the next chunk
  }
  if (pend_cid >= 0) store_pending();
}

// ---------------------------------------------------------------------------
// scan
// ---------------------------------------------------------------------------
template <int K, class TY>
__global__ __launch_bounds__(kThreads, 2) void mfma_scan_kernel(MfmaParams p) {
  constexpr int RB = K / 64;     // 16-row state blocks per wave
  constexpr int CB = kBV / 16;   // 16-column blocks per tile
  constexpr int KK = K / 32;     // 32-deep k-steps over the key dimension
  constexpr int KP = K + 8;
  constexpr int LP = kL + 8;
  // bf16(S)ᵀ is double-buffered (the readout of chunk n and the state update
  // writing chunk n+1's copy need no barrier between them); the low part
  // bf16(S − bf16(S))ᵀ is only read by the retrieval.
  __shared__ __attribute__((aligned(16))) uint16_t ShT[2][kBV * KP];
  __shared__ __attribute__((aligned(16))) uint16_t SlT[kBV * KP];
  __shared__ __attribute__((aligned(16))) uint16_t XbT[kBV * LP];  // bf16(X)ᵀ
  __shared__ __attribute__((aligned(16))) uint16_t XlT[kBV * LP];  // bf16(X − bf16(X))ᵀ
  __shared__ __attribute__((aligned(16))) uint16_t VpT[kBV * LP];  // bf16 V'ᵀ
  __shared__ float xes[kL], wrs[kL];  // written and read by one wave only

  const int tiles = p.V / kBV;
  const int BH = p.B * p.H;
  // XCD-aware: the `tiles` workgroups of one (b, h) get ids ≡ (mod 8).
  const int id = blockIdx.x;
  const int group = id / (8 * tiles), within = id % (8 * tiles);
  const int tile = within / 8, bh = group * 8 + within % 8;
  if (bh >= BH) return;
  const int b = bh / p.H, h = bh % p.H;
  const int j0 = tile * kBV;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, q4 = lane >> 4, k8 = 8 * q4;

  // The state tile in accumulator layout: wave w holds rows
  // [w·K/4, (w+1)·K/4) as RB row blocks × CB column blocks.
  f32x4 S[RB][CB];
  const float* sin = p.s_in + size_t(bh) * K * p.V;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = wave * (K / 4) + 16 * rb + 4 * q4 + r;
        S[rb][cb][r] = sin[size_t(d) * p.V + j0 + 16 * cb + r16];
      }
  // bf16 hi/lo copies of Sᵀ: the retrieval K·S cancels against v, so it
  // reads S to ~2⁻¹⁶; the readout Q·S reads the hi part only.
  auto write_state = [&](uint16_t* sh) {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int d = wave * (K / 4) + 16 * rb + 4 * q4;
        const f32x4& v = S[rb][cb];
        const uint32_t h01 = pk_bf16(v[0], v[1]), h23 = pk_bf16(v[2], v[3]);
        const uint32_t l01 = pk_bf16(v[0] - lo_f(h01), v[1] - hi_f(h01));
        const uint32_t l23 = pk_bf16(v[2] - lo_f(h23), v[3] - hi_f(h23));
        const int at = (16 * cb + r16) * KP + d;
        *reinterpret_cast<uint2*>(&sh[at]) = make_uint2(h01, h23);
        *reinterpret_cast<uint2*>(&SlT[at]) = make_uint2(l01, l23);
      }
  };
  write_state(ShT[0]);

  // Every global read of a chunk is issued one chunk ahead, right after the
  // phase that consumed the previous buffer, so the serial chain over chunks
  // never waits on HBM. Lane (wave w, r16, q4) reads token row 16w + r16.
  const int my_tok = 16 * wave + r16;
  uint4 kA[KK];             // K[my_tok][32kk + k8 …]                 (phase 1)
  float gcA, glA, erA, wrA;  // gate values of my_tok and G_last
  uint32_t vA[CB][2];       // V[16w + 4q4 + r][j0 + 16cb + r16], bf16 pairs
  uint4 tA[2], tlA[2];      // T hi/lo rows my_tok                    (phase 2)
  uint4 qA[KK], atA[2];     // Q row and attn row of my_tok           (phase 3a)
  uint4 kcA[RB][2];         // Kcᵀ rows of this wave's state rows     (phase 3b)

  const size_t tokstride = size_t(p.H);  // rows between consecutive tokens
  const size_t bh_row0 = size_t(b) * p.S * p.H + h;
  // Reads and writes are unconditional, with padded tokens' addresses
  // redirected to a zero row or a sink row: every iteration then issues the
  // same sequence of memory operations, which keeps the compiler's in-order
  // vmcnt waits exact across the loop instead of draining every prefetch.
  const float* zero32 = reinterpret_cast<const float*>(p.zero);
  auto load_k = [&](int n) {
    const size_t cid = (size_t(b) * p.N + n) * p.H + h;
    const int tok = n * kL + my_tok;
    const bool ok = tok < p.S;
    const size_t row = bh_row0 + size_t(tok) * tokstride;
    const uint16_t* kr = ok ? p.k + row * K + k8 : p.zero;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) kA[kk] = *reinterpret_cast<const uint4*>(kr + 32 * kk);
    gcA = p.gc[cid * kL + my_tok];
    glA = p.gc[cid * kL + kL - 1];
    erA = *(ok ? p.erase + row : zero32);
    wrA = *(ok ? p.write + row : zero32);
  };
  auto load_v = [&](int n) {
    const int t0 = n * kL + 16 * wave + 4 * q4;
    const uint16_t* vb = p.v + (bh_row0 + size_t(t0) * tokstride) * p.V + j0 + r16;
    const size_t vstride = tokstride * p.V;
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int r2 = 0; r2 < 2; ++r2) {
        const uint32_t x0 = *(t0 + 2 * r2 < p.S ? vb + (2 * r2) * vstride + 16 * cb : p.zero);
        const uint32_t x1 =
            *(t0 + 2 * r2 + 1 < p.S ? vb + (2 * r2 + 1) * vstride + 16 * cb : p.zero);
        vA[cb][r2] = x0 | (x1 << 16);
      }
  };
  auto load_t = [&](int n) {
    const size_t off = ((size_t(b) * p.N + n) * p.H + h) * kL * kL + size_t(my_tok) * kL + k8;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      tA[kk] = *reinterpret_cast<const uint4*>(p.T + off + 32 * kk);
      tlA[kk] = *reinterpret_cast<const uint4*>(p.Tlo + off + 32 * kk);
    }
  };
  auto load_q = [&](int n) {
    const int tok = n * kL + my_tok;
    const uint16_t* qr =
        tok < p.S ? p.q + (bh_row0 + size_t(tok) * tokstride) * K + k8 : p.zero;
#pragma unroll
    for (int kk = 0; kk < KK; ++kk) qA[kk] = *reinterpret_cast<const uint4*>(qr + 32 * kk);
    const size_t off = ((size_t(b) * p.N + n) * p.H + h) * kL * kL + size_t(my_tok) * kL + k8;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
      atA[kk] = *reinterpret_cast<const uint4*>(p.attn + off + 32 * kk);
  };
  auto load_kc = [&](int n) {
    const uint16_t* kc = p.KcT + ((size_t(b) * p.N + n) * p.H + h) * K * kL + k8;
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk)
        kcA[rb][kk] = *reinterpret_cast<const uint4*>(
            kc + size_t(wave * (K / 4) + 16 * rb + r16) * kL + 32 * kk);
  };
  auto as8 = [](const uint4& x) { return __builtin_bit_cast(bf16x8, x); };

  load_k(0);
  load_v(0);
  load_t(0);
  load_q(0);
  for (int n = 0; n < p.N; ++n) {
    const int tok0 = n * kL;
    const int nn = n + 1 < p.N ? n + 1 : n;  // the last chunk prefetches itself again
    const uint16_t* sh = ShT[n & 1];

    // Gates of this wave's tokens (read back by this wave only); G is 0
    // throughout when there is no forget gate.
    const float egA = __expf(gcA);
    const float egl = __expf(glA);
    if (q4 == 0) {
      xes[my_tok] = erA * egA;
      wrs[my_tok] = wrA;
    }

    // Phase 1: X = w⊙V − (e⊙e^G)⊙(K·S), token rows 16·wave…
    {
      f32x4 acc[CB];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          acc[cb] = mfma16(as8(kA[kk]), ld8(&sh[(16 * cb + r16) * KP + 32 * kk + k8]), acc[cb]);
          acc[cb] = mfma16(as8(kA[kk]), ld8(&SlT[(16 * cb + r16) * KP + 32 * kk + k8]), acc[cb]);
        }
      }
      float xe[4], wr[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        xe[r] = xes[16 * wave + 4 * q4 + r];
        wr[r] = wrs[16 * wave + 4 * q4 + r];
      }
      load_k(nn);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int j = 16 * cb + r16;
        float x[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float vv = (r & 1) ? hi_f(vA[cb][r >> 1]) : lo_f(vA[cb][r >> 1]);
          x[r] = wr[r] * vv - xe[r] * acc[cb][r];
        }
        const uint32_t h01 = pk_bf16(x[0], x[1]), h23 = pk_bf16(x[2], x[3]);
        const uint32_t l01 = pk_bf16(x[0] - lo_f(h01), x[1] - hi_f(h01));
        const uint32_t l23 = pk_bf16(x[2] - lo_f(h23), x[3] - hi_f(h23));
        *reinterpret_cast<uint2*>(&XbT[j * LP + 16 * wave + 4 * q4]) = make_uint2(h01, h23);
        *reinterpret_cast<uint2*>(&XlT[j * LP + 16 * wave + 4 * q4]) = make_uint2(l01, l23);
      }
      load_v(nn);
    }
    __syncthreads();

    // Phase 2: V' = T·X, with both factors as bf16 hi + lo parts: for a
    // chunk of near-identical keys T differences near-equal rows of X.
    {
      f32x4 acc[CB];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        acc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf16x8 xh = ld8(&XbT[(16 * cb + r16) * LP + 32 * kk + k8]);
          acc[cb] = mfma16(as8(tA[kk]), xh, acc[cb]);
          acc[cb] = mfma16(as8(tlA[kk]), xh, acc[cb]);
          acc[cb] = mfma16(as8(tA[kk]), ld8(&XlT[(16 * cb + r16) * LP + 32 * kk + k8]), acc[cb]);
        }
      }
      load_t(nn);
      load_kc(n);  // consumed in phase 3b, after phase 3a's MFMAs
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int j = 16 * cb + r16;
        *reinterpret_cast<uint2*>(&VpT[j * LP + 16 * wave + 4 * q4]) =
            make_uint2(pk_bf16(acc[cb][0], acc[cb][1]), pk_bf16(acc[cb][2], acc[cb][3]));
      }
    }
    __syncthreads();

    // Phase 3a: yᵀ = (Sᵀ·Qᵀ)⊙(scale·e^G) + V'ᵀ·attnᵀ. In this orientation
    // lane (r16, q4) holds four consecutive value columns of its own token
    // my_tok, so y leaves in 8- or 16-byte stores.
    {
      f32x4 qs[CB], av[CB];
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        qs[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
        av[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < KK; ++kk)
          qs[cb] = mfma16(ld8(&sh[(16 * cb + r16) * KP + 32 * kk + k8]), as8(qA[kk]), qs[cb]);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          av[cb] = mfma16(ld8(&VpT[(16 * cb + r16) * LP + 32 * kk + k8]), as8(atA[kk]), av[cb]);
      }
      load_q(nn);
      const int t = tok0 + my_tok;
      const float ysc = p.scale * egA;
      TY* yrow = t < p.S ? static_cast<TY*>(p.y) + (bh_row0 + size_t(t) * tokstride) * p.V + j0
                         : reinterpret_cast<TY*>(p.sink);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        float o[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) o[r] = ysc * qs[cb][r] + av[cb][r];
        TY* dst = yrow + 16 * cb + 4 * q4;
        if constexpr (sizeof(TY) == 2)
          *reinterpret_cast<uint2*>(dst) = make_uint2(pk_bf16(o[0], o[1]), pk_bf16(o[2], o[3]));
        else
          *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
      }
    }

    // Phase 3b: S ← e^{G_last}⊙S + (e^{G_last−G}⊙K)ᵀ·V'; its bf16 copy goes
    // to the other buffer, so the readout above needs no barrier.
    {
#pragma unroll
      for (int rb = 0; rb < RB; ++rb)
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          f32x4 acc = S[rb][cb];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] *= egl;
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
            acc = mfma16(as8(kcA[rb][kk]), ld8(&VpT[(16 * cb + r16) * LP + 32 * kk + k8]), acc);
          S[rb][cb] = acc;
        }
      write_state(ShT[(n + 1) & 1]);
    }
    __syncthreads();
  }

  float* sout = p.s_out + size_t(bh) * K * p.V;
#pragma unroll
  for (int rb = 0; rb < RB; ++rb)
#pragma unroll
    for (int cb = 0; cb < CB; ++cb)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = wave * (K / 4) + 16 * rb + 4 * q4 + r;
        sout[size_t(d) * p.V + j0 + 16 * cb + r16] = S[rb][cb][r];
      }
}

size_t region(size_t bytes) { return align_up(bytes, 256); }

}  // namespace

bool mfma_fwd_supported(const Dims& d, int qkv_dtype, int y_dtype) {
  (void)y_dtype;
  return qkv_dtype == DN_BF16 && (d.K == 64 || d.K == 128) && d.V % kBV == 0 && d.L == kL &&
         d.ew == 1 && d.ww == 1 && d.dw <= 1;
}

size_t mfma_fwd_workspace(const Dims& d) {
  const size_t G = size_t(d.B) * d.N * d.H;
  return 3 * region(G * kL * kL * 2) + region(G * kL * 4) + region(G * size_t(d.K) * kL * 2) +
         region(kZeroElems * 2) + region(size_t(kBV) * (d.V / kBV) * 4);
}

hipError_t mfma_fwd(const Dims& d, int y_dtype, const void* q, const void* k, const void* v,
                    const float* erase, const float* write, const float* g,
                    const float* state_in, void* y, float* state_out, void* ws,
                    hipStream_t stream) {
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
  char* base = static_cast<char*>(ws);
  p.T = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * kL * 2);
  p.Tlo = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * kL * 2);
  p.attn = reinterpret_cast<uint16_t*>(base);
  base += region(G * kL * kL * 2);
  p.gc = reinterpret_cast<float*>(base);
  base += region(G * kL * 4);
  p.KcT = reinterpret_cast<uint16_t*>(base);
  base += region(G * size_t(d.K) * kL * 2);
  p.zero = reinterpret_cast<uint16_t*>(base);
  base += region(kZeroElems * 2);
  p.sink = reinterpret_cast<uint16_t*>(base);

  {
    // Two resident workgroups per CU (LDS-bound) walk all chunk-heads.
    const int grid = int(std::min<size_t>(G, size_t(2) * device_cu_count()));
    ProfScope ps("dn_mfma_intra", stream);
#define DN_INTRA(KD, GT)                                                                   \
  hipLaunchKernelGGL((mfma_intra_kernel<KD, GT>), dim3(unsigned(grid)), dim3(kThreads), 0, \
                     stream, p, int(G))
    if (d.K == 128) {
      if (p.gated) DN_INTRA(128, true); else DN_INTRA(128, false);
    } else {
      if (p.gated) DN_INTRA(64, true); else DN_INTRA(64, false);
    }
#undef DN_INTRA
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const int tiles = d.V / kBV;
  const int BH = d.B * d.H;
  const unsigned blocks = unsigned(((BH + 7) / 8) * 8 * tiles);
  const bool yb = y_dtype == DN_BF16;
  ProfScope ps("dn_mfma_scan", stream);
#define DN_SCAN(KD, TY) \
  hipLaunchKernelGGL((mfma_scan_kernel<KD, TY>), dim3(blocks), dim3(kThreads), 0, stream, p)
  if (d.K == 128) {
    if (yb) DN_SCAN(128, bf16); else DN_SCAN(128, float);
  } else {
    if (yb) DN_SCAN(64, bf16); else DN_SCAN(64, float);
  }
#undef DN_SCAN
  return hipGetLastError();
}

}  // namespace dn
