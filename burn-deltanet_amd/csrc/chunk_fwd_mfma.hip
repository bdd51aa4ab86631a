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

#include "dn_common.hpp"

namespace dn {
namespace {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

constexpr int kL = 64;        // chunk length
constexpr int kThreads = 256;  // 4 waves
constexpr int kBV = 64;       // value columns per scan workgroup

__device__ inline f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ inline bf16x8 ld8(const uint16_t* p) { return *reinterpret_cast<const bf16x8*>(p); }

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
  float* gc;       // [G][64]
};

// ---------------------------------------------------------------------------
// intra
// ---------------------------------------------------------------------------
template <int K>
__global__ __launch_bounds__(kThreads) void mfma_intra_kernel(MfmaParams p) {
  constexpr int KP = K + 8;  // padded LDS row (bf16 elements)
  // The K/Q tiles are dead once the scores are formed; T and the merge
  // scratch reuse their space, which keeps two workgroups per CU.
  constexpr int kTileBytes = 2 * kL * KP * 2;
  constexpr int kSolveBytes = (kL * (kL + 1) + (kL / 2) * (kL / 2 + 1)) * 4;
  __shared__ __attribute__((aligned(16)))
  unsigned char stage[kTileBytes > kSolveBytes ? kTileBytes : kSolveBytes];
  uint16_t* Ks = reinterpret_cast<uint16_t*>(stage);
  uint16_t* Qs = Ks + kL * KP;
  float(*Tm)[kL + 1] = reinterpret_cast<float(*)[kL + 1]>(stage);  // T, fp32
  float(*Xs)[kL / 2 + 1] =
      reinterpret_cast<float(*)[kL / 2 + 1]>(stage + kL * (kL + 1) * 4);
  __shared__ float A[kL][kL + 1];  // strict-lower Akk, fp32
  __shared__ __attribute__((aligned(16))) uint16_t At[kL * (kL + 8)];  // attn, bf16
  __shared__ float gcs[kL], ers[kL];

  const int cid = blockIdx.x;
  const int h = cid % p.H, n = (cid / p.H) % p.N, b = cid / (p.H * p.N);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int tok0 = n * kL;

  // Stage the K and Q chunk tiles (zero past the sequence end).
  for (int idx = tid; idx < kL * K / 8; idx += kThreads) {
    const int row = idx / (K / 8), c8 = idx % (K / 8);
    const int tok = tok0 + row;
    bf16x8 kv = zero8(), qv = zero8();
    if (tok < p.S) {
      const size_t off = ((size_t(b) * p.S + tok) * p.H + h) * K + 8 * c8;
      kv = ld8(p.k + off);
      qv = ld8(p.q + off);
    }
    *reinterpret_cast<bf16x8*>(&Ks[row * KP + 8 * c8]) = kv;
    *reinterpret_cast<bf16x8*>(&Qs[row * KP + 8 * c8]) = qv;
  }
  // In-chunk cumulative gate and the erase gate, one token per lane.
  if (wave == 0) {
    const int tok = tok0 + lane;
    const size_t row = (size_t(b) * p.S + tok) * p.H + h;
    float gv = (p.gated && tok < p.S) ? p.g[row] : 0.f;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const float up = __shfl_up(gv, off, 64);
      if (lane >= off) gv += up;
    }
    gcs[lane] = gv;
    ers[lane] = tok < p.S ? p.erase[row] : 0.f;
    p.gc[size_t(cid) * kL + lane] = gv;
  }
  __syncthreads();

  // Akk = e ⊙ (K Kᵀ) ⊙ decay (strict lower), attn = scale (Q Kᵀ) ⊙ decay.
  {
    const int rb = wave;
    const int r16 = lane & 15, k8 = 8 * (lane >> 4);
    bf16x8 ak[K / 32], aq[K / 32];
#pragma unroll
    for (int kk = 0; kk < K / 32; ++kk) {
      ak[kk] = ld8(&Ks[(16 * rb + r16) * KP + 32 * kk + k8]);
      aq[kk] = ld8(&Qs[(16 * rb + r16) * KP + 32 * kk + k8]);
    }
    for (int cb = 0; cb < 4; ++cb) {
      const int j = 16 * cb + r16;
      if (cb > rb) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * rb + 4 * (lane >> 4) + r;
          A[i][j] = 0.f;
          At[i * (kL + 8) + j] = 0;
        }
        continue;
      }
      f32x4 acck = {0.f, 0.f, 0.f, 0.f}, accq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < K / 32; ++kk) {
        const bf16x8 bk = ld8(&Ks[(16 * cb + r16) * KP + 32 * kk + k8]);
        acck = mfma16(ak[kk], bk, acck);
        accq = mfma16(aq[kk], bk, accq);
      }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * rb + 4 * (lane >> 4) + r;
        const float decay = (j <= i) ? (p.gated ? __expf(gcs[i] - gcs[j]) : 1.f) : 0.f;
        A[i][j] = (j < i) ? ers[i] * acck[r] * decay : 0.f;
        At[i * (kL + 8) + j] = f32_to_bf16(p.scale * accq[r] * decay);
      }
    }
  }
  __syncthreads();

  // T: invert the four 16×16 diagonal blocks (one wave each, a lane per column).
  if (lane < 16) {
    const int base = 16 * wave, c = lane;
    float t[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) t[i] = (i == c) ? 1.f : 0.f;
#pragma unroll
    for (int i = 1; i < 16; ++i) {
      if (i > c) {
        float acc = 0.f;
#pragma unroll
        for (int k2 = 0; k2 < i; ++k2) acc += A[base + i][base + k2] * t[k2];
        t[i] = -acc;
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) Tm[base + i][base + c] = t[i];
  }
  // Zero everything above the block diagonal that the merges do not write.
  for (int idx = tid; idx < kL * kL; idx += kThreads) {
    const int i = idx / kL, j = idx % kL;
    if (j / 16 > i / 16) Tm[i][j] = 0.f;
  }
  __syncthreads();
  // 16 → 32: T₁₀ = −T₁₁ A₁₀ T₀₀ for the two 32-blocks.
  for (int idx = tid; idx < 2 * 256; idx += kThreads) {
    const int pb = idx / 256, i = (idx / 16) % 16, j = idx % 16;
    const int r0 = 32 * pb + 16, c0 = 32 * pb;
    float acc = 0.f;
    for (int k2 = j; k2 < 16; ++k2) acc += A[r0 + i][c0 + k2] * Tm[c0 + k2][c0 + j];
    Xs[16 * pb + i][j] = acc;
  }
  __syncthreads();
  for (int idx = tid; idx < 2 * 256; idx += kThreads) {
    const int pb = idx / 256, i = (idx / 16) % 16, j = idx % 16;
    const int r0 = 32 * pb + 16, c0 = 32 * pb;
    float acc = 0.f;
    for (int k2 = 0; k2 <= i; ++k2) acc += Tm[r0 + i][r0 + k2] * Xs[16 * pb + k2][j];
    Tm[r0 + i][c0 + j] = -acc;
  }
  __syncthreads();
  // 32 → 64: T[32:,:32] = −T[32:,32:] A[32:,:32] T[:32,:32].
  for (int idx = tid; idx < 32 * 32; idx += kThreads) {
    const int i = idx / 32, j = idx % 32;
    float acc = 0.f;
    for (int k2 = j; k2 < 32; ++k2) acc += A[32 + i][k2] * Tm[k2][j];
    Xs[i][j] = acc;
  }
  __syncthreads();
  for (int idx = tid; idx < 32 * 32; idx += kThreads) {
    const int i = idx / 32, j = idx % 32;
    float acc = 0.f;
    for (int k2 = 0; k2 <= i; ++k2) acc += Tm[32 + i][32 + k2] * Xs[k2][j];
    Tm[32 + i][j] = -acc;
  }
  __syncthreads();

  // Store T and attn as bf16, 16 values per lane.
  {
    const int row = tid / 4, c0 = 16 * (tid % 4);
    uint16_t* tdst = p.T + size_t(cid) * kL * kL + row * kL + c0;
    uint16_t* ldst = p.Tlo + size_t(cid) * kL * kL + row * kL + c0;
    uint16_t* adst = p.attn + size_t(cid) * kL * kL + row * kL + c0;
    alignas(16) uint16_t tv[16], tl[16];
#pragma unroll
    for (int c = 0; c < 16; ++c) {
      const float x = Tm[row][c0 + c];
      tv[c] = f32_to_bf16(x);
      tl[c] = f32_to_bf16(x - bf16_to_f32(tv[c]));
    }
    *reinterpret_cast<bf16x8*>(tdst) = *reinterpret_cast<const bf16x8*>(&tv[0]);
    *reinterpret_cast<bf16x8*>(tdst + 8) = *reinterpret_cast<const bf16x8*>(&tv[8]);
    *reinterpret_cast<bf16x8*>(ldst) = *reinterpret_cast<const bf16x8*>(&tl[0]);
    *reinterpret_cast<bf16x8*>(ldst + 8) = *reinterpret_cast<const bf16x8*>(&tl[8]);
    *reinterpret_cast<bf16x8*>(adst) = ld8(&At[row * (kL + 8) + c0]);
    *reinterpret_cast<bf16x8*>(adst + 8) = ld8(&At[row * (kL + 8) + c0 + 8]);
  }
}

// ---------------------------------------------------------------------------
// scan
// ---------------------------------------------------------------------------
template <int K, class TY>
__global__ __launch_bounds__(kThreads) void mfma_scan_kernel(MfmaParams p) {
  constexpr int RB = K / 64;     // 16-row state blocks per wave
  constexpr int CB = kBV / 16;   // 16-column blocks per tile
  constexpr int KP = K + 8;
  constexpr int LP = kL + 8;
  __shared__ __attribute__((aligned(16))) uint16_t KcT[K * LP];    // (e^{Gl−G}⊙K)ᵀ
  __shared__ __attribute__((aligned(16))) uint16_t ShT[kBV * KP];  // bf16(S)ᵀ
  __shared__ __attribute__((aligned(16))) uint16_t SlT[kBV * KP];  // bf16(S − bf16(S))ᵀ
  __shared__ __attribute__((aligned(16))) uint16_t XbT[kBV * LP];  // bf16(X)ᵀ
  __shared__ __attribute__((aligned(16))) uint16_t XlT[kBV * LP];  // bf16(X − bf16(X))ᵀ
  __shared__ __attribute__((aligned(16))) uint16_t VpT[kBV * LP];  // bf16 V'ᵀ
  __shared__ float egs[kL], xes[kL], wrs[kL];
  __shared__ float egl_s;

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
  auto write_state = [&]() {
#pragma unroll
    for (int rb = 0; rb < RB; ++rb)
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        const int d = wave * (K / 4) + 16 * rb + 4 * q4;
        uint16_t hi[4], lo[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          hi[r] = f32_to_bf16(S[rb][cb][r]);
          lo[r] = f32_to_bf16(S[rb][cb][r] - bf16_to_f32(hi[r]));
        }
        const int at = (16 * cb + r16) * KP + d;
        *reinterpret_cast<uint2*>(&ShT[at]) =
            make_uint2(uint32_t(hi[0]) | (uint32_t(hi[1]) << 16),
                       uint32_t(hi[2]) | (uint32_t(hi[3]) << 16));
        *reinterpret_cast<uint2*>(&SlT[at]) =
            make_uint2(uint32_t(lo[0]) | (uint32_t(lo[1]) << 16),
                       uint32_t(lo[2]) | (uint32_t(lo[3]) << 16));
      }
  };
  write_state();

  const size_t rowstride = size_t(p.H) * K;  // elements between tokens in q/k
  for (int n = 0; n < p.N; ++n) {
    const size_t cid = (size_t(b) * p.N + n) * p.H + h;
    const int tok0 = n * kL;
    const float glast = p.gated ? p.gc[cid * kL + kL - 1] : 0.f;
    // Phase 0: (e^{G_last−G}⊙K)ᵀ of the chunk into LDS; per-token gates.
    for (int idx = tid; idx < kL * K / 8; idx += kThreads) {
      const int row = idx / (K / 8), c8 = idx % (K / 8);
      const int tok = tok0 + row;
      uint4 kv = make_uint4(0u, 0u, 0u, 0u);
      if (tok < p.S)
        kv = *reinterpret_cast<const uint4*>(p.k + ((size_t(b) * p.S + tok) * p.H + h) * K +
                                             8 * c8);
      const float ec = p.gated ? __expf(glast - p.gc[cid * kL + row]) : 1.f;
      // Split the eight bf16 values with integer shifts (element reads of a
      // __bf16 vector are not reliable in this compiler).
      const uint32_t w4[4] = {kv.x, kv.y, kv.z, kv.w};
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        KcT[(8 * c8 + 2 * e) * LP + row] = f32_to_bf16(bf16_to_f32(uint16_t(w4[e])) * ec);
        KcT[(8 * c8 + 2 * e + 1) * LP + row] =
            f32_to_bf16(bf16_to_f32(uint16_t(w4[e] >> 16)) * ec);
      }
    }
    if (wave == 0) {
      const float gcv = p.gated ? p.gc[cid * kL + lane] : 0.f;
      const int tok = tok0 + lane;
      const size_t row = (size_t(b) * p.S + tok) * p.H + h;
      const float eg = p.gated ? __expf(gcv) : 1.f;
      egs[lane] = eg;
      xes[lane] = tok < p.S ? p.erase[row] * eg : 0.f;
      wrs[lane] = tok < p.S ? p.write[row] : 0.f;
      if (lane == 0) egl_s = p.gated ? __expf(glast) : 1.f;
    }
    __syncthreads();

    // Phase 1: X = w⊙V − (e⊙e^G)⊙(K·S), token rows 16·wave…
    {
      const int tok = tok0 + 16 * wave + r16;
      bf16x8 a[K / 32];
#pragma unroll
      for (int kk = 0; kk < K / 32; ++kk)
        a[kk] = tok < p.S ? ld8(p.k + (size_t(b) * p.S + tok) * rowstride + size_t(h) * K +
                                32 * kk + k8)
                          : zero8();
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < K / 32; ++kk) {
          acc = mfma16(a[kk], ld8(&ShT[(16 * cb + r16) * KP + 32 * kk + k8]), acc);
          acc = mfma16(a[kk], ld8(&SlT[(16 * cb + r16) * KP + 32 * kk + k8]), acc);
        }
        const int j = 16 * cb + r16;
        uint16_t xv[4], xl[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * wave + 4 * q4 + r;
          const int t = tok0 + i;
          const float vv = t < p.S ? bf16_to_f32(p.v[((size_t(b) * p.S + t) * p.H + h) * p.V +
                                                     j0 + j])
                                   : 0.f;
          const float x = wrs[i] * vv - xes[i] * acc[r];
          xv[r] = f32_to_bf16(x);
          xl[r] = f32_to_bf16(x - bf16_to_f32(xv[r]));
        }
        *reinterpret_cast<uint2*>(&XbT[j * LP + 16 * wave + 4 * q4]) =
            make_uint2(uint32_t(xv[0]) | (uint32_t(xv[1]) << 16),
                       uint32_t(xv[2]) | (uint32_t(xv[3]) << 16));
        *reinterpret_cast<uint2*>(&XlT[j * LP + 16 * wave + 4 * q4]) =
            make_uint2(uint32_t(xl[0]) | (uint32_t(xl[1]) << 16),
                       uint32_t(xl[2]) | (uint32_t(xl[3]) << 16));
      }
    }
    __syncthreads();

    // Phase 2: V' = T·X, with both factors as bf16 hi + lo parts: for a
    // chunk of near-identical keys T differences near-equal rows of X.
    {
      const uint16_t* Tc = p.T + cid * kL * kL;
      const uint16_t* Tl = p.Tlo + cid * kL * kL;
      bf16x8 a[2], al[2];
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        a[kk] = ld8(Tc + (16 * wave + r16) * kL + 32 * kk + k8);
        al[kk] = ld8(Tl + (16 * wave + r16) * kL + 32 * kk + k8);
      }
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          const bf16x8 xh = ld8(&XbT[(16 * cb + r16) * LP + 32 * kk + k8]);
          acc = mfma16(a[kk], xh, acc);
          acc = mfma16(al[kk], xh, acc);
          acc = mfma16(a[kk], ld8(&XlT[(16 * cb + r16) * LP + 32 * kk + k8]), acc);
        }
        const int j = 16 * cb + r16;
        uint16_t vp[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) vp[r] = f32_to_bf16(acc[r]);
        *reinterpret_cast<uint2*>(&VpT[j * LP + 16 * wave + 4 * q4]) =
            make_uint2(uint32_t(vp[0]) | (uint32_t(vp[1]) << 16),
                       uint32_t(vp[2]) | (uint32_t(vp[3]) << 16));
      }
    }
    __syncthreads();

    // Phase 3a: y = (scale·e^G)⊙(Q·S) + attn·V'.
    {
      const int tok = tok0 + 16 * wave + r16;
      const uint16_t* Ac = p.attn + cid * kL * kL;
      bf16x8 a[K / 32], at[2];
#pragma unroll
      for (int kk = 0; kk < K / 32; ++kk)
        a[kk] = tok < p.S ? ld8(p.q + (size_t(b) * p.S + tok) * rowstride + size_t(h) * K +
                                32 * kk + k8)
                          : zero8();
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) at[kk] = ld8(Ac + (16 * wave + r16) * kL + 32 * kk + k8);
#pragma unroll
      for (int cb = 0; cb < CB; ++cb) {
        f32x4 qs = {0.f, 0.f, 0.f, 0.f}, av = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kk = 0; kk < K / 32; ++kk)
          qs = mfma16(a[kk], ld8(&ShT[(16 * cb + r16) * KP + 32 * kk + k8]), qs);
#pragma unroll
        for (int kk = 0; kk < 2; ++kk)
          av = mfma16(at[kk], ld8(&VpT[(16 * cb + r16) * LP + 32 * kk + k8]), av);
        const int j = j0 + 16 * cb + r16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = 16 * wave + 4 * q4 + r;
          const int t = tok0 + i;
          if (t < p.S)
            st(static_cast<TY*>(p.y), ((size_t(b) * p.S + t) * p.H + h) * p.V + j,
               p.scale * egs[i] * qs[r] + av[r]);
        }
      }
    }
    __syncthreads();

    // Phase 3b: S ← e^{G_last}⊙S + (e^{G_last−G}⊙K)ᵀ·V'.
    {
      const float egl = egl_s;
#pragma unroll
      for (int rb = 0; rb < RB; ++rb) {
        const int d = wave * (K / 4) + 16 * rb + r16;
        bf16x8 a[2];
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) a[kk] = ld8(&KcT[d * LP + 32 * kk + k8]);
#pragma unroll
        for (int cb = 0; cb < CB; ++cb) {
          f32x4 acc = S[rb][cb];
#pragma unroll
          for (int r = 0; r < 4; ++r) acc[r] *= egl;
#pragma unroll
          for (int kk = 0; kk < 2; ++kk)
            acc = mfma16(a[kk], ld8(&VpT[(16 * cb + r16) * LP + 32 * kk + k8]), acc);
          S[rb][cb] = acc;
        }
      }
      write_state();
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
  return 3 * region(G * kL * kL * 2) + region(G * kL * 4);
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

  {
    ProfScope ps("dn_mfma_intra", stream);
    if (d.K == 128)
      hipLaunchKernelGGL(mfma_intra_kernel<128>, dim3(unsigned(G)), dim3(kThreads), 0, stream,
                         p);
    else
      hipLaunchKernelGGL(mfma_intra_kernel<64>, dim3(unsigned(G)), dim3(kThreads), 0, stream,
                         p);
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
