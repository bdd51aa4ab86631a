// The chunk-local gradients of the chunkwise WY form on CDNA4 matrix cores.
//
// combined_backward.rs:103-188 (WY and front-end terms), :240-319 (the
// per-chunk terms of the reverse walk) and :376-513 (both score backwards),
// for one chunk-head per workgroup (8 waves), given what the two MFMA scans
// leave behind: the state S₀ entering the chunk and the cotangent dS of the
// state leaving it (fp32), and the intra kernel's T, Tᵀ (bf16 hi + lo) and
// attnᵀ tiles. With X = w⊙V − kg·S₀ (so that V' = U − W·S₀ = T·X):
//
//   phase A  (a wave per 16 value columns)
//            X;  V' = T·X;  dV' = attnᵀ·dY + kc·dS;  dVw = Tᵀ·dV'
//            d_v = w⊙dVw, d_write from dVw⊙v
//   phase B  (a wave per 16 key channels; contractions over the value axis)
//            d_kc = V'·dSᵀ;  d_qr = dY·S₀ᵀ;  d_kg = −dVw·S₀ᵀ (= Tᵀ·dW with
//            dW = −dV'·S₀ᵀ);  Σ_v dS⊙S₀;  dattn = dY·V'ᵀ
//   phase C  dT = dV'·Xᵀ (= dU·Vwᵀ + dW·kgᵀ, without the cancellation of the
//            two terms);  dAkk = −tril(Tᵀ·dT·Tᵀ, −1) as (dTᵀ·T)ᵀ·Tᵀ
//   phase D  (a wave per 16 key channels) the score backward of the head
//            decay or of the per-channel block decay (BlockDecayPrim), the
//            gate terms and the reverse cumulative sum of d_g.
//
// Every product runs on v_mfma_f32_16x16x32_bf16 with fp32 intermediates as
// bf16 hi + lo parts (three MFMAs; two when one side is an exact bf16 input),
// which keeps the gradients at fp32-like accuracy. Intermediates pass between
// the phases through one LDS region that each phase re-carves.

#include <type_traits>

#include "dn_common.hpp"
#include "mfma_util.hpp"

namespace dn {
namespace {

constexpr int kL = 64;
constexpr int kW = 8;
constexpr int kNT = 64 * kW;
constexpr float kMaxExp = 48.f;  // MAX_EXPONENT, decay.rs:49

struct CbParams {
  int S, H, N, ew, ww;
  int gated;
  float scale;
  const uint16_t *q, *k, *v;
  const float *erase, *write, *g;
  const void* dy;
  const uint16_t *T, *Tlo, *Tt, *Ttl, *AtT;  // [G][64][64]
  const uint16_t* Kc;                        // [G][64][K] bf16(e^{G_last−G}⊙K)
  const uint16_t *Kg, *Kglo;                 // [G][64][K] e⊙e^G⊙K hi / lo (per-channel decay)
  const float* gc;                           // [G][64] in-chunk cumulative gate (per-head)
  const float* states;                       // [G][K][V]
  const float* ds_after;                     // [G][K][V]
  void *dq, *dk, *dv;
  float *derase, *dwrite, *dg;
  // The value axis in passes of at most 128 columns: this pass covers
  // columns voff … voff + V − 1 of rows vs wide (v, dO, the write gate, dv,
  // S₀ and dS). pass 0: the only pass; 1: the first of several, whose
  // value-summed outputs go to the fp32 partials; 2: a middle one, added to
  // them by atomics (nothing waits on them); 3: the last, which adds them and
  // stores.
  int vs, voff, pass;
  // head_k_dim 256 (KA = 2K, per-head gates): each value pass runs as two
  // launches, one per half of the key channels; phase A contracts over all
  // KA keys in both and only the first (koff = 0) stores its outputs. rpass:
  // the pass code (as `pass`) of the sums over key channels (d_g, a width-1
  // d_erase) across all the launches of a call; `pass` where KA = K.
  int koff, rpass;
  float *pq, *pk, *pe, *pg, *pw;  // partials of d_q, d_k, d_erase, d_g, width-1 d_write
  // Per-head gates over several passes: each thread's partial sums of dattn
  // and dT (16 fp32 per thread per chunk-head), which the passes before the
  // last hand on so that the last runs the score backward once.
  float* pda;
};

// A value-summed output (d_q, d_k, d_erase, d_g, a width-1 d_write): a sum
// over the value axis, so over the passes (CbParams::pass). The last pass
// reads the partial here, a round trip before the store, unless the caller
// loaded it ahead (st_last).
template <class T>
__device__ inline void st_sum(int pass, T* out, float* part, size_t i, float v) {
  if (pass == 1)
    part[i] = v;
  else if (pass == 2)
    atomicAdd(part + i, v);
  else
    st(out, i, pass == 3 ? v + part[i] : v);
}
// st_sum with the last pass's partial already in `pre` (0 when not the last).
template <class T>
__device__ inline void st_pre(int pass, T* out, float* part, size_t i, float v, float pre) {
  if (pass == 1)
    part[i] = v;
  else if (pass == 2)
    atomicAdd(part + i, v);
  else
    st(out, i, v + pre);
}

__device__ inline uint16_t bf_bits(float x) { return __builtin_bit_cast(uint16_t, (__bf16)x); }

// Four floats → packed bf16 hi parts and lo parts (8-byte LDS stores).
__device__ inline void split4(const float* f, uint2& h, uint2& l) {
  h = make_uint2(pk_bf16(f[0], f[1]), pk_bf16(f[2], f[3]));
  l = make_uint2(pk_bf16(f[0] - lo_f(h.x), f[1] - hi_f(h.x)),
                 pk_bf16(f[2] - lo_f(h.y), f[3] - hi_f(h.y)));
}

// v[0..15] summed over the 16 lanes that share lane/16; lane l receives the
// total of index l%16 (a halving exchange: 15 shuffles instead of 64).
__device__ inline float reduce16(const float (&v)[16], int lane) {
  float a[8], b[4], c[2];
  const bool u8 = lane & 8, u4 = lane & 4, u2 = lane & 2, u1 = lane & 1;
#pragma unroll
  for (int j = 0; j < 8; ++j)
    a[j] = (u8 ? v[8 + j] : v[j]) + __shfl_xor(u8 ? v[j] : v[8 + j], 8);
#pragma unroll
  for (int j = 0; j < 4; ++j)
    b[j] = (u4 ? a[4 + j] : a[j]) + __shfl_xor(u4 ? a[j] : a[4 + j], 4);
#pragma unroll
  for (int j = 0; j < 2; ++j)
    c[j] = (u2 ? b[2 + j] : b[j]) + __shfl_xor(u2 ? b[j] : b[2 + j], 2);
  return (u1 ? c[1] : c[0]) + __shfl_xor(u1 ? c[0] : c[1], 1);
}

// Materialises x in a register at this point: keeps the compiler from sinking
// an accumulation chain into the guarded store that consumes it, which would
// hold every partial term live until then.
__device__ inline void pin(float& x) { asm volatile("" : "+v"(x)); }
__device__ inline void pin(f32x4& x) { asm volatile("" : "+v"(x)); }

// Lanes 32…63 take b, lanes 0…31 keep a: one DPP move with a row mask. A
// per-lane select whose operand is a load let the compiler move the load into
// a branch for the lanes that use it, with a wait of its own.
__device__ inline float upper_half_take(float a, float b) {
  return __int_as_float(
      __builtin_amdgcn_update_dpp(__float_as_int(a), __float_as_int(b), 0xE4, 0xC, 0xF, false));
}

// v[0..3] summed over the 16 lanes that share lane/16; lane l receives the
// total of index l%4.
__device__ inline float reduce4(const float (&v)[4], int lane) {
  const bool u2 = lane & 2, u1 = lane & 1;
  float a[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
    a[j] = (u2 ? v[2 + j] : v[j]) + __shfl_xor(u2 ? v[j] : v[2 + j], 2);
  float c = (u1 ? a[1] : a[0]) + __shfl_xor(u1 ? a[0] : a[1], 1);
  c += __shfl_xor(c, 4);
  return c + __shfl_xor(c, 8);
}

// A 64×64 bf16 tile (global, row-major) → LDS with the permuted column order:
// thread tid loads 16-byte chunk tid (512 threads, one each), then stores it.
__device__ inline uint4 load_perm(const uint16_t* src, int tid) {
  return *reinterpret_cast<const uint4*>(src + (tid >> 3) * kL + 8 * (tid & 7));
}
__device__ inline void store_perm(uint16_t* R, int dst, const uint4& v, int tid) {
  const int row = tid >> 3, c8 = tid & 7;
  *reinterpret_cast<uint2*>(&R[dst + tile_at<kL>(row, perm_pos(8 * c8))]) = make_uint2(v.x, v.y);
  *reinterpret_cast<uint2*>(&R[dst + tile_at<kL>(row, perm_pos(8 * c8 + 4))]) =
      make_uint2(v.z, v.w);
}
__device__ inline void stage_perm(uint16_t* R, int dst, const uint16_t* src, int tid) {
  store_perm(R, dst, load_perm(src, tid), tid);
}

// The 16 lower-or-diagonal and upper 16×16 tiles of a 64×64 matrix, two per
// wave: tile t = wave + 8u is (t/4, t%4).

// LASTP (per-head gates, the last of several value passes): the partials
// of the value-summed outputs are loaded at the start of phase D, so their
// round trip overlaps the score backward instead of preceding each store.
// EARLY (per-head gates, the passes before the last): dattn and dT are sums
// over the value axis, and everything after them is linear in them, so these
// passes add their partial sums to p.pda and stop after phase C's first
// product; the score backward (the rest of phase C and phase D's scores) runs
// once, in the last pass, on the summed dattn and dT. They still store their
// share of the value-summed gradients (phase B's terms).
// KA: the head_k_dim of the tensors; phase A's contractions run over all KA
// keys and phases B–D over K of them from channel p.koff on (KA = 2K: the
// key halves of head_k_dim 256, per-head gates).
template <int K, int V, bool PC, class TG, bool LASTP = false, bool EARLY = false, int KA = K>
__global__ __launch_bounds__(kNT) void mfma_chunk_bwd_kernel(CbParams p) {
  static_assert(!(LASTP && PC), "the per-channel last pass reads its partials at the stores");
  static_assert(KA == K || (KA == 2 * K && !PC), "key halves: per-head gates");
  constexpr int KS = KA;  // row stride of q, k, the states and the key-channel outputs
  // The states and state cotangents in row groups of four, [G][K/4][V][4]
  // (mfma_bwd_scans' g4, at head_k_dim 256), else [G][K][V].
  constexpr bool G4 = KA == 256;
  static_assert(!(EARLY && (PC || LASTP)), "partial score sums: per-head gates, not the last pass");
  constexpr bool F32DY = std::is_same<TG, float>::value;
  constexpr int TT = kL * kL, TK = kL * K, TKA = kL * KA, TV = kL * V;
  constexpr int OFF_A1 = 4 * TV > 8 * TT ? 4 * TV : 8 * TT;
  constexpr int RBIG = OFF_A1 + 4 * TT;
  static_assert(5 * TT + (PC ? 3 : 1) * TKA <= RBIG, "phase-A operands fit");
  static_assert((F32DY ? 6 : 5) * TV <= RBIG, "phase-B operands fit");
  static_assert(4 * TT + 2 * TK <= OFF_A1, "score operands fit");
  constexpr int GP = K + 4;  // fp32 row pitch of the per-channel cumulative gate
  // Carvings of R (bf16 elements):
  //  A  T hi/lo, Tᵀ hi/lo (permuted), attnᵀ (permuted), kg (hi/lo), kc
  constexpr int oTh = 0, oTl = TT, oTth = 2 * TT, oTtl = 3 * TT, oAt = 4 * TT, oKop = 5 * TT,
                oKgl = 5 * TT + TK, oKc = PC ? 5 * TT + 2 * TK : 5 * TT;
  //  B  V' hi/lo, dVw hi/lo, dY hi(/lo)
  constexpr int oVh = 0, oVl = TV, oWh = 2 * TV, oWl = 3 * TV, oYh = 4 * TV, oYl = 5 * TV;
  //  C  X hi/lo, dV' hi/lo; dAqk as [i][j] and [j][i] (hi/lo) at OFF_A1 until the end
  constexpr int oXh = 0, oXl = TV, oDh = 2 * TV, oDl = 3 * TV;
  constexpr int oA1h = OFF_A1, oA1l = OFF_A1 + TT, oA1th = OFF_A1 + 2 * TT,
                oA1tl = OFF_A1 + 3 * TT;
  //     then T and Tᵀ again, dTᵀ (permuted over dT's rows), M₁ = Tᵀ·dT
  constexpr int oDTh = 4 * TT, oDTl = 5 * TT, oM1h = 6 * TT, oM1l = 7 * TT;
  //  D  dAkk as [i][j] and [j][i] (hi/lo); Kᵀ, Qᵀ
  constexpr int oA0h = 0, oA0l = TT, oA0th = 2 * TT, oA0tl = 3 * TT, oKC = 4 * TT,
                oQC = 4 * TT + TK;
  __shared__ __attribute__((aligned(16))) uint16_t R[RBIG];
  __shared__ __attribute__((aligned(16))) float Gc[PC ? kL * GP : kL];
  __shared__ float er_s[kL], wr_s[kL], eg_s[kL], ec_s[kL];
  __shared__ float racc[3][kL];  // row sums: d_write, d_erase, d_g (per-head)
  __shared__ float cacc[K];      // per-channel decay: d(G_last) per channel

  const int cid = blockIdx.x;
  const int h = cid % p.H, n = (cid / p.H) % p.N, b = cid / (p.H * p.N);
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, g4 = lane >> 4, k8 = 8 * g4;
  const int tok0 = n * kL;
  const int valid = min(kL, p.S - tok0);
  const size_t row0 = size_t(b) * p.S * p.H + h + size_t(tok0) * p.H;
  auto row_of = [&](int t) { return row0 + size_t(t) * p.H; };
  // Global reads are unconditional: a row past the sequence end reads the
  // chunk's last row (valid ≥ 1) and the value is then dropped. A load under
  // a lane guard becomes a branch of its own with a full wait on every load
  // in flight, which serialised the staging.
  auto rowc = [&](int t) { return row_of(min(t, valid - 1)); };
  const size_t o64 = size_t(cid) * kL * kL, oLK = size_t(cid) * kL * K;
  const int VS = p.vs, vo = p.voff;  // row stride and first column of the value axis
  // Row-major: element (row, column) at S0[row·VS + column]; in row groups
  // of four at S0[(row/4·VS + column)·4 + row%4] (the pass's first column
  // is then 4·vo floats in).
  const float* S0 = p.states + size_t(cid) * KS * VS + (G4 ? 4 * vo : vo);
  const float* dSa = p.ds_after + size_t(cid) * KS * VS + (G4 ? 4 * vo : vo);
  // This launch's first key channel (phases B–D), and whether it stores the
  // outputs of phase A and accumulates the value-summed dattn and dT.
  const int koff = KA == K ? 0 : p.koff;
  const bool store_a = koff == 0;
  const TG* dy = static_cast<const TG*>(p.dy);
  const bool gated = PC || p.gated;
  auto rowi = [&](int ib, int r) { return 16 * ib + 4 * g4 + r; };
  // Row of the value reduce16 leaves in this lane (index 4·ib + r).
  const int red_row = 16 * (r16 >> 2) + 4 * g4 + (r16 & 3);

  // ---- staging -----------------------------------------------------------
  // The gate and tile loads are issued together and written to LDS (one
  // round trip); phase A's operand loads follow, in flight across the
  // cumulative sum and the barriers. Loads complete in order, so issuing the
  // phase-A loads first would make every LDS write wait for them too.
  float e0 = 0.f, w0 = 0.f, gct = 0.f, gl = 0.f;
  if (tid < kL) {
    // Index rowc(t) is in bounds at either gate width.
    e0 = p.erase[rowc(tid)];
    w0 = p.write[rowc(tid)];
    if constexpr (!PC) {
      if (gated) {
        gct = p.gc[size_t(cid) * kL + tid];
        gl = p.gc[size_t(cid) * kL + kL - 1];
      }
    }
  }
  constexpr int KPART = kNT / K, RUN = kL / KPART;  // per-channel cumulative sum
  float vals[PC ? RUN : 1];
  if constexpr (PC) {
    const int d = tid % K, part = tid / K;
#pragma unroll
    for (int t = 0; t < RUN; ++t) {
      const int tt = part * RUN + t;
      const float x = p.g[rowc(tt) * K + d];
      vals[t] = tt < valid ? x : 0.f;
    }
  }

  constexpr int NKR = kL * KA / 8 / kNT;  // 16-byte chunks per thread of a [64][KA] tile
  static_assert(NKR * kNT * 8 == kL * KA, "K-wide staging assumes whole rounds");
  uint4 tp[5], tk[PC ? 3 : 1][NKR];
  tp[0] = load_perm(p.T + o64, tid);
  tp[1] = load_perm(p.Tlo + o64, tid);
  tp[2] = load_perm(p.Tt + o64, tid);
  tp[3] = load_perm(p.Ttl + o64, tid);
  tp[4] = load_perm(p.AtT + o64, tid);
#pragma unroll
  for (int m = 0; m < NKR; ++m) {
    const int idx = tid + kNT * m, row = idx / (KA / 8), c8 = idx % (KA / 8);
    if constexpr (PC) {
      const size_t o = oLK + size_t(row) * K + 8 * c8;
      tk[0][m] = *reinterpret_cast<const uint4*>(p.Kg + o);
      tk[1][m] = *reinterpret_cast<const uint4*>(p.Kglo + o);
      tk[2][m] = *reinterpret_cast<const uint4*>(p.Kc + o);
    } else {
      const uint4 x = *reinterpret_cast<const uint4*>(p.k + rowc(row) * KS + 8 * c8);
      tk[0][m] = row < valid ? x : make_uint4(0u, 0u, 0u, 0u);
    }
  }
  if (tid < kL) {
    const int t = tid;
    const bool ok = t < valid;
    er_s[t] = (ok && p.ew == 1) ? e0 : 0.f;
    wr_s[t] = (ok && p.ww == 1) ? w0 : 0.f;
    if constexpr (!PC) {
      Gc[t] = gct;
      eg_s[t] = gated ? __expf(gct) : 1.f;
      ec_s[t] = gated ? __expf(gl - gct) : 1.f;
    }
    racc[0][t] = racc[1][t] = racc[2][t] = 0.f;
  }
  store_perm(R, oTh, tp[0], tid);
  store_perm(R, oTl, tp[1], tid);
  store_perm(R, oTth, tp[2], tid);
  store_perm(R, oTtl, tp[3], tid);
  store_perm(R, oAt, tp[4], tid);
#pragma unroll
  for (int m = 0; m < NKR; ++m) {
    const int idx = tid + kNT * m, row = idx / (KA / 8), c8 = idx % (KA / 8);
    const int at = tile_at<KA>(row, 8 * c8);
    *reinterpret_cast<uint4*>(&R[oKop + at]) = tk[0][m];
    if constexpr (PC) {
      *reinterpret_cast<uint4*>(&R[oKgl + at]) = tk[1][m];
      *reinterpret_cast<uint4*>(&R[oKc + at]) = tk[2][m];
    }
  }

  // ---- phase A's global operands -------------------------------------------
  const bool vwave = wave < V / 16;
  const int col = 16 * wave + r16;  // this lane's value column in phase A
  // S₀ and dS for PDEP k-steps at a time: all of them at head_k_dim ≤ 128;
  // at 256 the first four, each register set reloaded with the k-step four
  // ahead once its fragments are split.
  constexpr int KAS = KA / 32, PDEP = KAS > 4 ? 4 : KAS;
  float pS[PDEP][8], pD[PDEP][8], vv[4][4], wv[4][4], dyv[2][8];
  auto load_sd = [&](float (&dst)[8], const float* src, int s) {
    if constexpr (G4) {
      // rows 32s + k8 … +3 and +4 … +7 of column col: two 16-byte loads
      const float4* b = reinterpret_cast<const float4*>(src) + size_t(8 * s + 2 * g4) * VS + col;
      const float4 lo = b[0], hi = b[VS];
      dst[0] = lo.x; dst[1] = lo.y; dst[2] = lo.z; dst[3] = lo.w;
      dst[4] = hi.x; dst[5] = hi.y; dst[6] = hi.z; dst[7] = hi.w;
    } else {
#pragma unroll
      for (int t = 0; t < 8; ++t) dst[t] = src[size_t(32 * s + k8 + t) * VS + col];
    }
  };
  if (vwave) {
    // S₀ and dS rows 32·s + 8·(lane/16) + t of this lane's column (B operands
    // of kg·S₀ and kc·dS).
    if constexpr (G4) {
#pragma unroll
      for (int s = 0; s < PDEP; ++s) {
        load_sd(pS[s], S0, s);
        load_sd(pD[s], dSa, s);
      }
    } else {
#pragma unroll
      for (int s = 0; s < PDEP; ++s)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          pS[s][t] = S0[size_t(32 * s + k8 + t) * VS + col];
          pD[s][t] = dSa[size_t(32 * s + k8 + t) * VS + col];
        }
    }
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = rowi(ib, r);
        const float x = bf16_to_f32(p.v[rowc(i) * VS + vo + col]);
        vv[ib][r] = i < valid ? x : 0.f;
      }
    if (p.ww != 1) {
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = rowi(ib, r);
          const float x = p.write[rowc(i) * VS + vo + col];
          wv[ib][r] = i < valid ? x : 0.f;
        }
    } else {
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int r = 0; r < 4; ++r) wv[ib][r] = 0.f;
    }
    // dY in the permuted token order of the attnᵀ fragments: token 4q+e /
    // 16+4q+e of each 32-token step at position 8q+e / 8q+4+e.
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const int t = 32 * kk + (e < 4 ? 4 * g4 + e : 16 + 4 * g4 + e - 4);
        const float x = ld(dy, rowc(t) * VS + vo + col);
        dyv[kk][e] = t < valid ? x : 0.f;
      }
  }
  for (int c = tid; c < K; c += kNT) cacc[c] = 0.f;
  if constexpr (PC) {
    // G = in-chunk cumulative sum of g per channel (KPART lanes per channel).
    const int d = tid % K, part = tid / K;
    float acc = 0.f;
#pragma unroll
    for (int t = 0; t < RUN; ++t) {
      acc += vals[t];
      vals[t] = acc;
    }
    Gc[(part * RUN + RUN - 1) * GP + d] = acc;
    __syncthreads();
    float carry = 0.f;
    for (int pp = 0; pp < part; ++pp) carry += Gc[(pp * RUN + RUN - 1) * GP + d];
    __syncthreads();
#pragma unroll
    for (int t = 0; t < RUN; ++t) Gc[(part * RUN + t) * GP + d] = vals[t] + carry;
  }
  __syncthreads();

  // ---- phase A: value columns ---------------------------------------------
  f32x4 X[4], dV[4], Vn[4], dW[4];
  if (vwave) {
    if (p.ww == 1)
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int r = 0; r < 4; ++r) wv[ib][r] = wr_s[rowi(ib, r)];
    // X = w⊙V − kg·S₀ (S₀ as hi + lo parts; per-head: k exact, e·e^G per row).
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) X[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < KAS; ++s) {
      uint4 sh, sl;
      split8(pS[s % PDEP], sh, sl);
      if (s + PDEP < KAS) {
        // (a scheduling barrier: hoisted to the staging, these reloads
        // spilled the loaded values there, each load waited for in turn)
        __builtin_amdgcn_sched_barrier(0);
        load_sd(pS[s % PDEP], S0, s + PDEP);
      }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        const int at = tile_at<KA>(16 * ib + r16, 32 * s + k8);
        const uint4 a = ld8u(&R[oKop + at]);
        X[ib] = mfma16(a, sh, X[ib]);
        X[ib] = mfma16(a, sl, X[ib]);
        if constexpr (PC) X[ib] = mfma16(ld8u(&R[oKgl + at]), sh, X[ib]);
      }
    }
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = rowi(ib, r);
        const float sc = PC ? 1.f : er_s[i] * eg_s[i];
        X[ib][r] = vv[ib][r] * wv[ib][r] - sc * X[ib][r];
      }
    // V' = T·X (hi + lo parts of both).
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) Vn[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint4 xh = frag_hi(X[2 * kk], X[2 * kk + 1]);
      const uint4 xl = frag_lo(X[2 * kk], X[2 * kk + 1], xh);
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        if (kk > (ib >> 1)) continue;  // T is lower triangular
        const int at = tile_at<kL>(16 * ib + r16, 32 * kk + k8);
        const uint4 th = ld8u(&R[oTh + at]), tl = ld8u(&R[oTl + at]);
        Vn[ib] = mfma16(th, xh, Vn[ib]);
        Vn[ib] = mfma16(tl, xh, Vn[ib]);
        Vn[ib] = mfma16(th, xl, Vn[ib]);
      }
    }
    // dV' = attnᵀ·dY + kc·dS (dY fragments: token 4q+e / 16+4q+e of each
    // 32-token step at position 8q+e / 8q+4+e, the permuted order).
    uint4 yh[2], yl[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) split8(dyv[kk], yh[kk], yl[kk]);
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) {
      dV[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        if (kk < (ib >> 1)) continue;  // attnᵀ is upper triangular
        const uint4 a = ld8u(&R[oAt + tile_at<kL>(16 * ib + r16, 32 * kk + k8)]);
        dV[ib] = mfma16(a, yh[kk], dV[ib]);
        if constexpr (F32DY) dV[ib] = mfma16(a, yl[kk], dV[ib]);
      }
    }
    {
      f32x4 kd[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) kd[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < KAS; ++s) {
        uint4 dh, dl;
        split8(pD[s % PDEP], dh, dl);
        if (s + PDEP < KAS) {
          __builtin_amdgcn_sched_barrier(0);
          load_sd(pD[s % PDEP], dSa, s + PDEP);
        }
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          const uint4 a = ld8u(&R[oKc + tile_at<KA>(16 * ib + r16, 32 * s + k8)]);
          kd[ib] = mfma16(a, dh, kd[ib]);
          kd[ib] = mfma16(a, dl, kd[ib]);
        }
      }
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int r = 0; r < 4; ++r) dV[ib][r] += (PC ? 1.f : ec_s[rowi(ib, r)]) * kd[ib][r];
    }
    // dVw = Tᵀ·dV'.
#pragma unroll
    for (int ib = 0; ib < 4; ++ib) dW[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      const uint4 vh = frag_hi(dV[2 * kk], dV[2 * kk + 1]);
      const uint4 vl = frag_lo(dV[2 * kk], dV[2 * kk + 1], vh);
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        if (kk < (ib >> 1)) continue;  // Tᵀ is upper triangular
        const int at = tile_at<kL>(16 * ib + r16, 32 * kk + k8);
        const uint4 th = ld8u(&R[oTth + at]), tl = ld8u(&R[oTtl + at]);
        dW[ib] = mfma16(th, vh, dW[ib]);
        dW[ib] = mfma16(tl, vh, dW[ib]);
        dW[ib] = mfma16(th, vl, dW[ib]);
      }
    }
    // d_v = w⊙dVw; d_write = dVw⊙v, summed over the value axis for width 1.
    TG* gv = static_cast<TG*>(p.dv);
    float rs[16];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = rowi(ib, r);
        if (store_a && i < valid) st(gv, row_of(i) * VS + vo + col, dW[ib][r] * wv[ib][r]);
        rs[4 * ib + r] = dW[ib][r] * vv[ib][r];
        if (p.ww != 1 && store_a && i < valid)
          p.dwrite[row_of(i) * VS + vo + col] = rs[4 * ib + r];
      }
    if (p.ww == 1) atomicAdd(&racc[0][red_row], reduce16(rs, lane));
  }
  // dY rows for LDS, then phase B's global operands: S₀ and dS rows of this
  // lane's key channel.
  constexpr int NY = kL * V / 8 / kNT;  // 16-byte chunks of dY rows per thread
  static_assert(NY * kNT * 8 == kL * V, "dY staging assumes whole rounds");
  float ydat[NY][8];
#pragma unroll
  for (int m = 0; m < NY; ++m) {
    const int idx = tid + kNT * m, i = idx / (V / 8), c8 = idx % (V / 8);
    if constexpr (F32DY) {
      const float4* src = reinterpret_cast<const float4*>(dy + rowc(i) * VS + vo + 8 * c8);
      float4 a = src[0], b2 = src[1];
      if (i >= valid) a = b2 = make_float4(0.f, 0.f, 0.f, 0.f);
      ydat[m][0] = a.x; ydat[m][1] = a.y; ydat[m][2] = a.z; ydat[m][3] = a.w;
      ydat[m][4] = b2.x; ydat[m][5] = b2.y; ydat[m][6] = b2.z; ydat[m][7] = b2.w;
    } else {
      uint4 v = *reinterpret_cast<const uint4*>(reinterpret_cast<const uint16_t*>(dy) +
                                                rowc(i) * VS + vo + 8 * c8);
      if (i >= valid) v = make_uint4(0u, 0u, 0u, 0u);
      unpack8(v, ydat[m]);
    }
  }
  const bool kwave = wave < K / 16;
  const int c = 16 * wave + r16;  // this lane's key channel in phases B and D
  float bS[V / 32][8], bD[V / 32][8], eA[4][4];
  if (kwave) {
    if constexpr (G4) {
      // row koff + c: element (koff + c)%4 of each column's row group
      const int row = koff + c;
      const size_t o = size_t(row >> 2) * VS * 4 + (row & 3);
#pragma unroll
      for (int s = 0; s < V / 32; ++s)
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          bS[s][t] = S0[o + size_t(32 * s + k8 + t) * 4];
          bD[s][t] = dSa[o + size_t(32 * s + k8 + t) * 4];
        }
    } else {
#pragma unroll
      for (int s = 0; s < V / 32; ++s) {
        const float4* s0r = reinterpret_cast<const float4*>(S0 + size_t(koff + c) * VS + 32 * s + k8);
        const float4* dsr = reinterpret_cast<const float4*>(dSa + size_t(koff + c) * VS + 32 * s + k8);
        *reinterpret_cast<float4*>(bS[s]) = s0r[0];
        *reinterpret_cast<float4*>(bS[s] + 4) = s0r[1];
        *reinterpret_cast<float4*>(bD[s]) = dsr[0];
        *reinterpret_cast<float4*>(bD[s] + 4) = dsr[1];
      }
    }
  }
  __syncthreads();

  // ---- V', dVw and dY rows into LDS ---------------------------------------
  if (vwave) {
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int at = tile_at<V>(rowi(ib, r), col);
        const uint16_t vh = bf_bits(Vn[ib][r]), wh = bf_bits(dW[ib][r]);
        R[oVh + at] = vh;
        R[oVl + at] = bf_bits(Vn[ib][r] - bf16_to_f32(vh));
        R[oWh + at] = wh;
        R[oWl + at] = bf_bits(dW[ib][r] - bf16_to_f32(wh));
      }
  }
#pragma unroll
  for (int m = 0; m < NY; ++m) {
    const int idx = tid + kNT * m, i = idx / (V / 8), c8 = idx % (V / 8);
    const int at = tile_at<V>(i, 8 * c8);
    uint4 hh, ll;
    split8(ydat[m], hh, ll);
    *reinterpret_cast<uint4*>(&R[oYh + at]) = hh;
    if constexpr (F32DY) *reinterpret_cast<uint4*>(&R[oYl + at]) = ll;
  }
  __syncthreads();

  // ---- phase B: key channels; contractions over the value axis ------------
  f32x4 dkA[4], dqA[4], dkeA[4];
  float dgA[4][4], degl = 0.f;
  if (kwave) {
    f32x4 aKc[4], aQr[4], aKg[4];
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
      aKc[ib] = aQr[ib] = aKg[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < V / 32; ++s) {
#pragma unroll
      for (int t = 0; t < 8; ++t) degl += bS[s][t] * bD[s][t];
      uint4 sh, sl, dh, dl;
      split8(bS[s], sh, sl);
      split8(bD[s], dh, dl);
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        const int at = tile_at<V>(16 * ib + r16, 32 * s + k8);
        const uint4 vh = ld8u(&R[oVh + at]), vl = ld8u(&R[oVl + at]);
        aKc[ib] = mfma16(vh, dh, aKc[ib]);
        aKc[ib] = mfma16(vl, dh, aKc[ib]);
        aKc[ib] = mfma16(vh, dl, aKc[ib]);
        const uint4 yh = ld8u(&R[oYh + at]);
        aQr[ib] = mfma16(yh, sh, aQr[ib]);
        aQr[ib] = mfma16(yh, sl, aQr[ib]);
        if constexpr (F32DY) aQr[ib] = mfma16(ld8u(&R[oYl + at]), sh, aQr[ib]);
        const uint4 wh = ld8u(&R[oWh + at]), wl = ld8u(&R[oWl + at]);
        aKg[ib] = mfma16(wh, sh, aKg[ib]);
        aKg[ib] = mfma16(wl, sh, aKg[ib]);
        aKg[ib] = mfma16(wh, sl, aKg[ib]);
      }
    }
    degl += __shfl_xor(degl, 16);
    degl += __shfl_xor(degl, 32);
    // The scan's cotangents through the gates (combined_backward.rs:284-313):
    // d_k = d_kc⊙e^{G_last−G}, d_q = d_qr⊙e^G, d_ke = d_kg⊙e^G (their d_G
    // pieces follow in phase D, where K and Q are staged).
    const float gl_c = PC ? Gc[(kL - 1) * GP + c] : 0.f;
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = rowi(ib, r);
        float eg, ec;
        if constexpr (PC) {
          const float gci = Gc[i * GP + c];
          eg = __expf(gci);
          ec = __expf(gl_c - gci);
        } else {
          eg = eg_s[i];
          ec = ec_s[i];
        }
        dkA[ib][r] = aKc[ib][r] * ec;
        dqA[ib][r] = aQr[ib][r] * eg;
        dkeA[ib][r] = -aKg[ib][r] * eg;
      }
  }
  // dattn = dY·V'ᵀ on the lower tiles.
  f32x4 dat[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int t = wave + 8 * u, ti = t >> 2, tj = t & 3;
    dat[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (tj <= ti) {
#pragma unroll
      for (int s = 0; s < V / 32; ++s) {
        const int aa = tile_at<V>(16 * ti + r16, 32 * s + k8);
        const int ab = tile_at<V>(16 * tj + r16, 32 * s + k8);
        const uint4 yh = ld8u(&R[oYh + aa]);
        const uint4 bh = ld8u(&R[oVh + ab]), bl = ld8u(&R[oVl + ab]);
        dat[u] = mfma16(yh, bh, dat[u]);
        dat[u] = mfma16(yh, bl, dat[u]);
        if constexpr (F32DY) dat[u] = mfma16(ld8u(&R[oYl + aa]), bh, dat[u]);
      }
    }
  }
  // The earlier passes' dattn and dT partial sums (this thread's 16 slots).
  float* const da = PC || !p.pda ? nullptr : p.pda + (size_t(cid) * kNT + tid) * 16;
  f32x4 pda_r[4];
  if constexpr (!PC) {
    if (LASTP || (EARLY && p.pass == 2 && store_a))
#pragma unroll
      for (int j = 0; j < 4; ++j) pda_r[j] = reinterpret_cast<const f32x4*>(da)[j];
  }
  __syncthreads();
  // Per-channel erase gate at the lane's rows, for phase D: loaded here so
  // that phase B does not hold it, its latency covered by phase C. One load
  // whose index depends on the gate width (a load inside a branch would be
  // waited for where the branch joins).
  if (PC && kwave)
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = rowi(ib, r);
        const float x = p.erase[p.ew == 1 ? rowc(i) : rowc(i) * K + c];
        eA[ib][r] = i < valid ? x : 0.f;
      }

  // ---- X, dV' rows and the dAqk layouts into LDS --------------------------
  if (vwave) {
#pragma unroll
    for (int ib = 0; ib < 4; ++ib)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int at = tile_at<V>(rowi(ib, r), col);
        const uint16_t xh = bf_bits(X[ib][r]), dh = bf_bits(dV[ib][r]);
        R[oXh + at] = xh;
        R[oXl + at] = bf_bits(X[ib][r] - bf16_to_f32(xh));
        R[oDh + at] = dh;
        R[oDl + at] = bf_bits(dV[ib][r] - bf16_to_f32(dh));
      }
  }
  if constexpr (!PC) {
    if (LASTP || (EARLY && p.pass == 2 && store_a))
#pragma unroll
      for (int u = 0; u < 2; ++u) dat[u] += pda_r[u];
  }
  if constexpr (EARLY) {
    if (store_a)
#pragma unroll
      for (int u = 0; u < 2; ++u) reinterpret_cast<f32x4*>(da)[u] = dat[u];
  }
  // dAqk = tril(dattn) (per-head decay: ⊙ e^{Gᵢ−Gⱼ}, the head mask) as
  // [i][j] and as [j][i] (per-head: times the readout scale).
  if constexpr (!EARLY) {
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = wave + 8 * u, ti = t >> 2, tj = t & 3;
      const int j = 16 * tj + r16;
      float f[4], ft[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * ti + 4 * g4 + r;
        float val = 0.f;
        if (j <= i) {
          val = dat[u][r];
          if (!PC && gated) val *= __expf(Gc[i] - Gc[j]);
        }
        f[r] = val;
        ft[r] = PC ? val : val * p.scale;
        const int at = tile_at<kL>(i, j);
        const uint16_t vh = bf_bits(val);
        R[oA1h + at] = vh;
        R[oA1l + at] = bf_bits(val - bf16_to_f32(vh));
      }
      uint2 hh, ll;
      split4(ft, hh, ll);
      const int at = tile_at<kL>(j, 16 * ti + 4 * g4);
      *reinterpret_cast<uint2*>(&R[oA1th + at]) = hh;
      *reinterpret_cast<uint2*>(&R[oA1tl + at]) = ll;
    }
  }
  __syncthreads();

  // ---- phase C: dT = dV'·Xᵀ (strict lower) --------------------------------
  f32x4 dTt[2];
#pragma unroll
  for (int u = 0; u < 2; ++u) {
    const int t = wave + 8 * u, ti = t >> 2, tj = t & 3;
    dTt[u] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (tj <= ti) {
#pragma unroll
      for (int s = 0; s < V / 32; ++s) {
        const int aa = tile_at<V>(16 * ti + r16, 32 * s + k8);
        const int ab = tile_at<V>(16 * tj + r16, 32 * s + k8);
        const uint4 ah = ld8u(&R[oDh + aa]), al = ld8u(&R[oDl + aa]);
        const uint4 bh = ld8u(&R[oXh + ab]), bl = ld8u(&R[oXl + ab]);
        dTt[u] = mfma16(ah, bh, dTt[u]);
        dTt[u] = mfma16(al, bh, dTt[u]);
        dTt[u] = mfma16(ah, bl, dTt[u]);
      }
    }
  }
  __syncthreads();
  if constexpr (!PC) {
    if (LASTP || (EARLY && p.pass == 2 && store_a))
#pragma unroll
      for (int u = 0; u < 2; ++u) dTt[u] += pda_r[2 + u];
  }
  if constexpr (EARLY) {
    if (store_a)
#pragma unroll
      for (int u = 0; u < 2; ++u) reinterpret_cast<f32x4*>(da)[2 + u] = dTt[u];
  } else {
    // dTᵀ with dT's row index permuted (it is the contraction index of dTᵀ·T);
    // T and Tᵀ staged again.
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = wave + 8 * u, ti = t >> 2, tj = t & 3;
      float f[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int a = 16 * ti + 4 * g4 + r, bcol = 16 * tj + r16;
        f[r] = bcol < a ? dTt[u][r] : 0.f;
      }
      uint2 hh, ll;
      split4(f, hh, ll);
      const int at = tile_at<kL>(16 * tj + r16, 32 * (ti >> 1) + 8 * g4 + 4 * (ti & 1));
      *reinterpret_cast<uint2*>(&R[oDTh + at]) = hh;
      *reinterpret_cast<uint2*>(&R[oDTl + at]) = ll;
    }
    stage_perm(R, oTh, p.T + o64, tid);
    stage_perm(R, oTl, p.Tlo + o64, tid);
    stage_perm(R, oTth, p.Tt + o64, tid);
    stage_perm(R, oTtl, p.Ttl + o64, tid);
    __syncthreads();
    // M₁ᵀ = dTᵀ·T (all 16 tiles), stored as M₁ with its column index permuted.
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = wave + 8 * u, bt = t >> 2, it = t & 3;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        // dTᵀ and Tᵀ are upper triangular: k-step 0 (j < 32) vanishes for
        // row blocks 2 and 3 of either.
        if (kk < (max(bt, it) >> 1)) continue;
        const int aa = tile_at<kL>(16 * bt + r16, 32 * kk + k8);
        const int ab = tile_at<kL>(16 * it + r16, 32 * kk + k8);
        const uint4 ah = ld8u(&R[oDTh + aa]), al = ld8u(&R[oDTl + aa]);
        const uint4 bh = ld8u(&R[oTth + ab]), bl = ld8u(&R[oTtl + ab]);
        acc = mfma16(ah, bh, acc);
        acc = mfma16(al, bh, acc);
        acc = mfma16(ah, bl, acc);
      }
      float f[4] = {acc[0], acc[1], acc[2], acc[3]};
      uint2 hh, ll;
      split4(f, hh, ll);
      const int at = tile_at<kL>(16 * it + r16, 32 * (bt >> 1) + 8 * g4 + 4 * (bt & 1));
      *reinterpret_cast<uint2*>(&R[oM1h + at]) = hh;
      *reinterpret_cast<uint2*>(&R[oM1l + at]) = ll;
    }
    __syncthreads();
    // dAkk = −tril(M₁·Tᵀ, −1); T[j][b] vanishes for b > j.
    f32x4 dak[2];
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = wave + 8 * u, ti = t >> 2, tj = t & 3;
      dak[u] = f32x4{0.f, 0.f, 0.f, 0.f};
      if (tj <= ti) {
#pragma unroll
        for (int kk = 0; kk < 2; ++kk) {
          if (kk > (tj >> 1)) continue;
          const int aa = tile_at<kL>(16 * ti + r16, 32 * kk + k8);
          const int ab = tile_at<kL>(16 * tj + r16, 32 * kk + k8);
          const uint4 ah = ld8u(&R[oM1h + aa]), al = ld8u(&R[oM1l + aa]);
          const uint4 bh = ld8u(&R[oTh + ab]), bl = ld8u(&R[oTl + ab]);
          dak[u] = mfma16(ah, bh, dak[u]);
          dak[u] = mfma16(al, bh, dak[u]);
          dak[u] = mfma16(ah, bl, dak[u]);
        }
      }
    }
    __syncthreads();
    // dAkk (per-head decay: ⊙ the head mask) as [i][j] and as [j][i]
    // (per-head: times the erase gate of row i); Kᵀ and Qᵀ.
#pragma unroll
    for (int u = 0; u < 2; ++u) {
      const int t = wave + 8 * u, ti = t >> 2, tj = t & 3;
      const int j = 16 * tj + r16;
      float ft[4];
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int i = 16 * ti + 4 * g4 + r;
        float val = 0.f;
        if (j < i) {
          val = -dak[u][r];
          if (!PC && gated) val *= __expf(Gc[i] - Gc[j]);
        }
        ft[r] = PC ? val : val * er_s[i];
        const int at = tile_at<kL>(i, j);
        const uint16_t vh = bf_bits(val);
        R[oA0h + at] = vh;
        R[oA0l + at] = bf_bits(val - bf16_to_f32(vh));
      }
      uint2 hh, ll;
      split4(ft, hh, ll);
      const int at = tile_at<kL>(j, 16 * ti + 4 * g4);
      *reinterpret_cast<uint2*>(&R[oA0th + at]) = hh;
      *reinterpret_cast<uint2*>(&R[oA0tl + at]) = ll;
    }
  }
  for (int idx = tid; idx < kL * K / 8; idx += kNT) {
    const int i = idx / (K / 8), c8 = idx % (K / 8);
    uint4 kv = *reinterpret_cast<const uint4*>(p.k + rowc(i) * KS + koff + 8 * c8);
    uint4 qv = *reinterpret_cast<const uint4*>(p.q + rowc(i) * KS + koff + 8 * c8);
    if (i >= valid) kv = qv = make_uint4(0u, 0u, 0u, 0u);
    const uint32_t kw[4] = {kv.x, kv.y, kv.z, kv.w}, qw[4] = {qv.x, qv.y, qv.z, qv.w};
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int at = tile_at<kL>(8 * c8 + e, i);
      R[oKC + at] = uint16_t(kw[e >> 1] >> (16 * (e & 1)));
      R[oQC + at] = uint16_t(qw[e >> 1] >> (16 * (e & 1)));
    }
  }
  __syncthreads();

  // ---- phase D: score backward, gates, stores -----------------------------
  // The last pass's partials: d_q and d_k at this lane's 16 rows and channel;
  // the row sums (d_write, d_erase, d_g) at row `lane` (stored by wave 0).
  float pre_q[16], pre_k[16], pre_w = 0.f, pre_e = 0.f, pre_g = 0.f;
  if constexpr (LASTP) {
    if (kwave) {
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const size_t at = rowc(rowi(ib, r)) * KS + koff + c;
          pre_q[4 * ib + r] = p.pq[at];
          pre_k[4 * ib + r] = p.pk[at];
        }
    }
    if (wave == 0) {
      const size_t at = rowc(lane);
      if (p.ww == 1) pre_w = p.pw[at];
      // (key halves: the sums over key channels go through st_sum(rpass))
      if constexpr (KA == K) {
        pre_e = p.pe[at];
        if (gated) pre_g = p.pg[at];
      }
    }
  }
  if (kwave) {
    TG* gq = static_cast<TG*>(p.dq);
    TG* gk = static_cast<TG*>(p.dk);
    // d_G of the scan (combined_backward.rs:284-313): −d_carry + (d_qr⊙qs +
    // d_kg⊙ke)⊙e^G = −dkA⊙k + dqA⊙q·scale + dkeA⊙k⊙e with phase B's
    // accumulators, and d(G_last) = Σ_i d_carry + (Σ_v dS⊙S₀)·e^{G_last}.
    if (gated) {
      float carry = 0.f, rowv[16];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        const uint2 k4 = *reinterpret_cast<const uint2*>(&R[oKC + tile_at<kL>(c, 16 * ib + 4 * g4)]);
        const uint2 q4 = *reinterpret_cast<const uint2*>(&R[oQC + tile_at<kL>(c, 16 * ib + 4 * g4)]);
        const float kv[4] = {lo_f(k4.x), hi_f(k4.x), lo_f(k4.y), hi_f(k4.y)};
        const float qv[4] = {lo_f(q4.x), hi_f(q4.x), lo_f(q4.y), hi_f(q4.y)};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float e = PC ? eA[ib][r] : er_s[rowi(ib, r)];
          const float dcarry = dkA[ib][r] * kv[r];
          const float val = -dcarry + dqA[ib][r] * qv[r] * p.scale + dkeA[ib][r] * kv[r] * e;
          carry += dcarry;
          if constexpr (PC) dgA[ib][r] = val;
          rowv[4 * ib + r] = val;
        }
      }
      if constexpr (PC) {
        carry += __shfl_xor(carry, 16);
        carry += __shfl_xor(carry, 32);
        if (g4 == 0) cacc[c] = carry + degl * __expf(Gc[(kL - 1) * GP + c]);
      } else {
        atomicAdd(&racc[2][red_row], reduce16(rowv, lane));
        // d(G_last) of the whole head: Σ d_carry + Σ_channels (dS⊙S₀)·e^{G_last}.
        float tot = carry + (g4 == 0 ? degl * eg_s[kL - 1] : 0.f);
#pragma unroll
        for (int m = 32; m >= 1; m >>= 1) tot += __shfl_xor(tot, m);
        if (lane == 0) atomicAdd(&racc[2][kL - 1], tot);
      }
    }
    if constexpr (EARLY) {
      // the score backward runs in the last pass
    } else if constexpr (!PC) {
      // head_scores_backward (combined_backward.rs:376-416) with drkk = dAkk⊙M,
      // drqk = dAqk⊙M: d_ke += drkk·K, d_qs += drqk·K, d_k += drkkᵀ·ke +
      // drqkᵀ·qs. The d_G term Σⱼ d_diff[i][j] − d_diff[j][i] of
      // d_diff = (dAkk⊙KeKᵀ + dAqk⊙QsKᵀ)⊙M equals, per row, Σ_c of
      // ke⊙(drkk·K) + qs⊙(drqk·K) − k⊙(drkkᵀ·ke + drqkᵀ·qs).
      f32x4 SK1[4], SQ1[4], SK2[4], SQ2[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
        SK1[ib] = SQ1[ib] = SK2[ib] = SQ2[ib] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const uint4 kb = ld8u(&R[oKC + tile_at<kL>(c, 32 * s + k8)]);
        const uint4 qb = ld8u(&R[oQC + tile_at<kL>(c, 32 * s + k8)]);
#pragma unroll
        for (int ib = 0; ib < 4; ++ib) {
          const int at = tile_at<kL>(16 * ib + r16, 32 * s + k8);
          if (s <= (ib >> 1)) {
            SK1[ib] = mfma16(ld8u(&R[oA0h + at]), kb, SK1[ib]);
            SK1[ib] = mfma16(ld8u(&R[oA0l + at]), kb, SK1[ib]);
            SQ1[ib] = mfma16(ld8u(&R[oA1h + at]), kb, SQ1[ib]);
            SQ1[ib] = mfma16(ld8u(&R[oA1l + at]), kb, SQ1[ib]);
          }
          if (s >= (ib >> 1)) {
            SK2[ib] = mfma16(ld8u(&R[oA0th + at]), kb, SK2[ib]);
            SK2[ib] = mfma16(ld8u(&R[oA0tl + at]), kb, SK2[ib]);
            SQ2[ib] = mfma16(ld8u(&R[oA1th + at]), qb, SQ2[ib]);
            SQ2[ib] = mfma16(ld8u(&R[oA1tl + at]), qb, SQ2[ib]);
          }
        }
      }
      float rowv[16];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        float kv[4], qv[4];
        {
          const uint2 k4 = *reinterpret_cast<const uint2*>(&R[oKC + tile_at<kL>(c, 16 * ib + 4 * g4)]);
          const uint2 q4 = *reinterpret_cast<const uint2*>(&R[oQC + tile_at<kL>(c, 16 * ib + 4 * g4)]);
          kv[0] = lo_f(k4.x); kv[1] = hi_f(k4.x); kv[2] = lo_f(k4.y); kv[3] = hi_f(k4.y);
          qv[0] = lo_f(q4.x); qv[1] = hi_f(q4.x); qv[2] = lo_f(q4.y); qv[3] = hi_f(q4.y);
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = rowi(ib, r);
          dkeA[ib][r] += SK1[ib][r];
          dqA[ib][r] += SQ1[ib][r];
          dkA[ib][r] += SK2[ib][r] + SQ2[ib][r];
          rowv[4 * ib + r] = er_s[i] * kv[r] * SK1[ib][r] + p.scale * qv[r] * SQ1[ib][r] -
                             kv[r] * (SK2[ib][r] + SQ2[ib][r]);
        }
      }
      if (gated) atomicAdd(&racc[2][red_row], reduce16(rowv, lane));
    } else {
      // channel_scores_backward (combined_backward.rs:421-513): per row block
      // pb with reference row r = 16·pb + 8, row factors e^{min(G[i]−G[r], 48)}
      // and column factors k[j]·e^{min(G[r]−G[j], 48)} (zero past block pb).
      // The row factors' gate (erase for the dAkk half of the lanes, the
      // readout scale for the dAqk half), loaded one row block ahead.
      auto gate8 = [&](int pb, float* e8) {
        const int i0 = 16 * pb + (k8 & 15);
#pragma unroll
        for (int t = 0; t < 8; ++t) {
          const int i = i0 + t;
          const float x = p.erase[p.ew == 1 ? rowc(i) : rowc(i) * K + c];
          e8[t] = upper_half_take(i < valid ? x : 0.f, p.scale);  // g4 ≥ 2: the readout scale
        }
      };
      float ecur[8];
      gate8(0, ecur);
#pragma unroll
      for (int pb = 0; pb < 4; ++pb) {
        float enext[8];
        if (pb < 3) gate8(pb + 1, enext);
        const float gref = Gc[(16 * pb + 8) * GP + c];
        // d(ke⊙rf), d(qs⊙rf) of the block's rows = dAkk, dAqk rows · colb.
        f32x4 drke = {0.f, 0.f, 0.f, 0.f}, drq = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s = 0; s < 2; ++s) {
          if (s > (pb >> 1)) continue;
          float kf[8], cb[8];
          unpack8(ld8u(&R[oKC + tile_at<kL>(c, 32 * s + k8)]), kf);
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int j = 32 * s + k8 + t;
            cb[t] = (j >> 4) <= pb ? kf[t] * __expf(fminf(gref - Gc[j * GP + c], kMaxExp)) : 0.f;
          }
          uint4 bh, bl;
          split8(cb, bh, bl);
          const int at = tile_at<kL>(16 * pb + r16, 32 * s + k8);
          const uint4 a0h = ld8u(&R[oA0h + at]), a1h = ld8u(&R[oA1h + at]);
          drke = mfma16(a0h, bh, drke);
          drke = mfma16(ld8u(&R[oA0l + at]), bh, drke);
          drke = mfma16(a0h, bl, drke);
          drq = mfma16(a1h, bh, drq);
          drq = mfma16(ld8u(&R[oA1l + at]), bh, drq);
          drq = mfma16(a1h, bl, drq);
        }
        // dcol[j][c] = Σ_{i∈pb} dAkk[i][j]·(ke⊙rf)[i][c] + dAqk[i][j]·(qs⊙rf)[i][c]
        // as one 32-deep step: positions 0..15 the dAkk rows, 16..31 the dAqk rows.
        uint4 rh, rl;
        {
          const bool isq = g4 >= 2;
          const int i0 = 16 * pb + (k8 & 15);
          float xf[8], rv[8];
          unpack8(ld8u(&R[(isq ? oQC : oKC) + tile_at<kL>(c, i0)]), xf);
#pragma unroll
          for (int t = 0; t < 8; ++t) {
            const int i = i0 + t;
            const float rf = __expf(fminf(Gc[i * GP + c] - gref, kMaxExp));
            rv[t] = xf[t] * ecur[t] * rf;
          }
          split8(rv, rh, rl);
        }
        f32x4 dcol[4];
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          dcol[jb] = f32x4{0.f, 0.f, 0.f, 0.f};
          if (jb > pb) continue;
          const int at = tile_at<kL>(16 * jb + r16, 16 * pb + (k8 & 15));
          const uint4 ah = ld8u(&R[(g4 >= 2 ? oA1th : oA0th) + at]);
          const uint4 al = ld8u(&R[(g4 >= 2 ? oA1tl : oA0tl) + at]);
          dcol[jb] = mfma16(ah, rh, dcol[jb]);
          dcol[jb] = mfma16(al, rh, dcol[jb]);
          dcol[jb] = mfma16(ah, rl, dcol[jb]);
        }
        // The block's rows: d_ke, d_qs through the row factor; d_G of its
        // exponent where the clamp does not bind.
        float drsum = 0.f;
        {
          float kv[4], qv[4];
          const uint2 k4 = *reinterpret_cast<const uint2*>(&R[oKC + tile_at<kL>(c, 16 * pb + 4 * g4)]);
          const uint2 q4 = *reinterpret_cast<const uint2*>(&R[oQC + tile_at<kL>(c, 16 * pb + 4 * g4)]);
          kv[0] = lo_f(k4.x); kv[1] = hi_f(k4.x); kv[2] = lo_f(k4.y); kv[3] = hi_f(k4.y);
          qv[0] = lo_f(q4.x); qv[1] = hi_f(q4.x); qv[2] = lo_f(q4.y); qv[3] = hi_f(q4.y);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = rowi(pb, r);
            const float arg = Gc[i * GP + c] - gref;
            const float rf = __expf(fminf(arg, kMaxExp));
            dkeA[pb][r] += drke[r] * rf;
            dqA[pb][r] += drq[r] * rf;
            const float drow = drke[r] * kv[r] * eA[pb][r] + drq[r] * qv[r] * p.scale;
            const float dra = arg < kMaxExp ? drow * rf : 0.f;
            dgA[pb][r] += dra;
            drsum += dra;
          }
        }
        // The columns: d_k through the column factor, d_G of its exponent.
        float dref = 0.f;
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          if (jb > pb) continue;
          const uint2 k4 = *reinterpret_cast<const uint2*>(&R[oKC + tile_at<kL>(c, 16 * jb + 4 * g4)]);
          const float kv[4] = {lo_f(k4.x), hi_f(k4.x), lo_f(k4.y), hi_f(k4.y)};
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int j = rowi(jb, r);
            const float arg = gref - Gc[j * GP + c];
            const float ce = __expf(fminf(arg, kMaxExp));
            dkA[jb][r] += dcol[jb][r] * ce;
            const float tv = arg < kMaxExp ? dcol[jb][r] * kv[r] * ce : 0.f;
            dgA[jb][r] -= tv;
            dref += tv;
          }
        }
        // d_G of the reference row: the column exponents' total minus the row
        // exponents' (both are relative to it).
        float tot = dref - drsum;
        tot += __shfl_xor(tot, 16);
        tot += __shfl_xor(tot, 32);
        if (g4 == 2) dgA[pb][0] += tot;
        // Only this iteration adds to row block pb's d_q and d_ke: store d_q,
        // fold d_ke⊙e into d_k and emit d_erase now, which frees their
        // registers for the blocks that follow.
        {
          const uint2 k4 = *reinterpret_cast<const uint2*>(&R[oKC + tile_at<kL>(c, 16 * pb + 4 * g4)]);
          const float kv[4] = {lo_f(k4.x), hi_f(k4.x), lo_f(k4.y), hi_f(k4.y)};
          float rde[4];
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const int i = rowi(pb, r);
            const bool ok = i < valid;
            if (ok) st_sum(p.pass, gq, p.pq, row_of(i) * KS + koff + c, dqA[pb][r] * p.scale);
            dkA[pb][r] += dkeA[pb][r] * eA[pb][r];
            rde[r] = dkeA[pb][r] * kv[r];
            if (p.ew != 1 && ok) st_sum(p.pass, p.derase, p.pe, row_of(i) * KS + koff + c, rde[r]);
          }
          if (p.ew == 1) {
            const float tot4 = reduce4(rde, lane);
            if ((lane & 12) == 0) atomicAdd(&racc[1][rowi(pb, lane & 3)], tot4);
          }
        }
#pragma unroll
        for (int jb = 0; jb < 4; ++jb) {
          pin(dkA[jb]);
#pragma unroll
          for (int r = 0; r < 4; ++r) pin(dgA[jb][r]);
        }
        if (pb < 3)
#pragma unroll
          for (int t = 0; t < 8; ++t) ecur[t] = enext[t];
      }
    }
    // Front end (combined_backward.rs:153-188) and the stores (the
    // per-channel branch has stored d_q and d_erase block by block).
    if constexpr (PC) {
#pragma unroll
      for (int ib = 0; ib < 4; ++ib)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = rowi(ib, r);
          if (i < valid) st_sum(p.pass, gk, p.pk, row_of(i) * KS + koff + c, dkA[ib][r]);
        }
    } else {
      float rde[16];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        const uint2 k4 = *reinterpret_cast<const uint2*>(&R[oKC + tile_at<kL>(c, 16 * ib + 4 * g4)]);
        const float kv[4] = {lo_f(k4.x), hi_f(k4.x), lo_f(k4.y), hi_f(k4.y)};
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = rowi(ib, r);
          const bool ok = i < valid;
          if (ok) {
            const size_t at = row_of(i) * KS + koff + c;
            const float vq = dqA[ib][r] * p.scale, vk = dkA[ib][r] + dkeA[ib][r] * er_s[i];
            if constexpr (LASTP) {
              st_pre(p.pass, gq, p.pq, at, vq, pre_q[4 * ib + r]);
              st_pre(p.pass, gk, p.pk, at, vk, pre_k[4 * ib + r]);
            } else {
              st_sum(p.pass, gq, p.pq, at, vq);
              st_sum(p.pass, gk, p.pk, at, vk);
            }
          }
          rde[4 * ib + r] = dkeA[ib][r] * kv[r];
          if (p.ew != 1 && ok)
            st_sum(p.pass, p.derase, p.pe, row_of(i) * KS + koff + c, rde[4 * ib + r]);
        }
      }
      if (p.ew == 1) atomicAdd(&racc[1][red_row], reduce16(rde, lane));
    }
  }
  if constexpr (PC) {
    // d_g = the reverse cumulative sum over the chunk of d_G (row L−1 also
    // takes d(G_last)): within the lane's 4 rows, across the 4 lanes of its
    // column, then across the 16-row blocks.
    if (kwave) {
      float tot[4], after[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
#pragma unroll
        for (int r = 2; r >= 0; --r) dgA[ib][r] += dgA[ib][r + 1];
        tot[ib] = dgA[ib][0];
      }
      float blk[4];
#pragma unroll
      for (int ib = 0; ib < 4; ++ib) {
        const float t0 = __shfl(tot[ib], r16), t1 = __shfl(tot[ib], r16 + 16),
                    t2 = __shfl(tot[ib], r16 + 32), t3 = __shfl(tot[ib], r16 + 48);
        after[ib] = (g4 < 1 ? t1 : 0.f) + (g4 < 2 ? t2 : 0.f) + (g4 < 3 ? t3 : 0.f);
        blk[ib] = t0 + t1 + t2 + t3;
      }
      float carry = cacc[c];
#pragma unroll
      for (int ib = 3; ib >= 0; --ib) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int i = rowi(ib, r);
          if (i < valid)
            st_sum(p.pass, p.dg, p.pg, row_of(i) * KS + koff + c, dgA[ib][r] + after[ib] + carry);
        }
        carry += blk[ib];
      }
    }
    __syncthreads();
  } else {
    __syncthreads();
    if (gated && wave == 0) {
      float v = racc[2][lane];
#pragma unroll
      for (int off = 1; off < 64; off <<= 1) {
        const float t = __shfl_down(v, off);
        if (lane + off < 64) v += t;
      }
      if (lane < valid) {
        if constexpr (LASTP && KA == K)
          st_pre(p.pass, p.dg, p.pg, row_of(lane), v, pre_g);
        else
          st_sum(p.rpass, p.dg, p.pg, row_of(lane), v);
      }
    }
  }
  if (tid < valid) {
    if constexpr (LASTP) {
      if (p.ww == 1 && store_a) st_pre(p.pass, p.dwrite, p.pw, row_of(tid), racc[0][tid], pre_w);
      if (p.ew == 1) {
        if constexpr (KA == K)
          st_pre(p.pass, p.derase, p.pe, row_of(tid), racc[1][tid], pre_e);
        else
          st_sum(p.rpass, p.derase, p.pe, row_of(tid), racc[1][tid]);
      }
    } else {
      if (p.ww == 1 && store_a) st_sum(p.pass, p.dwrite, p.pw, row_of(tid), racc[0][tid]);
      if (p.ew == 1) st_sum(p.rpass, p.derase, p.pe, row_of(tid), racc[1][tid]);
    }
  }
}

}  // namespace

// head_v_dim 64 or 128 in one pass; above 128 in passes of 128 columns, the
// last of 64 when head_v_dim is an odd multiple of 64. head_k_dim 256 with
// per-head gates: each pass as two launches over the halves of the keys.
bool mfma_chunk_bwd_supported(const Dims& d, int qkv_dtype) {
  if (!(mfma_fwd_supported(d, qkv_dtype, DN_BF16) && d.V % 64 == 0)) return false;
  if (d.K == 256) return d.dw <= 1 && d.ew == 1 && d.ww == 1;
  return d.K <= 128;
}

// The fp32 partial sums of the value-summed gradients across the passes:
// per (token, head) d_q, d_k (K each), d_erase (ew), d_g (dw) and d_write
// (1 when its width is 1). None for a single pass of a single launch (at
// head_k_dim 256 the key halves add d_g and d_erase across launches).
size_t mfma_chunk_bwd_partials(const Dims& d) {
  if (d.V <= 128 && d.K <= 128) return 0;
  const size_t rows = size_t(d.B) * d.S * d.H;
  const bool pc = d.dw == d.K && d.K > 1;
  const size_t G = size_t(d.B) * d.N * d.H;
  return align_up(rows * (2 * d.K + d.ew + d.dw + (d.ww == 1 ? 1 : 0)) * sizeof(float), 256) +
         (pc || d.V <= 128 ? 0 : G * kNT * 16 * sizeof(float));  // dattn and dT partial sums
}

hipError_t mfma_chunk_bwd(const Dims& d, int grad_dtype, const void* dy, const void* q,
                          const void* k, const void* v, const float* erase, const float* write,
                          const float* g, const float* states, const float* ds_after, void* dq,
                          void* dk, void* dv, float* derase, float* dwrite, float* dg,
                          const MfmaTiles& tiles, float* partials, hipStream_t stream, bool g4) {
  // The chunk-local kernels read the row-group layout exactly at head_k_dim 256.
  if (g4 != (d.K == 256)) return hipErrorInvalidValue;
  CbParams p;
  p.S = d.S;
  p.H = d.H;
  p.N = d.N;
  p.ew = d.ew;
  p.ww = d.ww;
  p.gated = d.dw > 0;
  p.scale = d.scale;
  p.q = static_cast<const uint16_t*>(q);
  p.k = static_cast<const uint16_t*>(k);
  p.v = static_cast<const uint16_t*>(v);
  p.erase = erase;
  p.write = write;
  p.g = g;
  p.dy = dy;
  p.T = tiles.T;
  p.Tlo = tiles.Tlo;
  p.Tt = tiles.Tt;
  p.Ttl = tiles.Ttl;
  p.AtT = tiles.AtT;
  p.Kc = tiles.Kc;
  p.Kg = tiles.Kg;
  p.Kglo = tiles.Kglo;
  p.gc = tiles.gc;
  p.states = states;
  p.ds_after = ds_after;
  p.dq = dq;
  p.dk = dk;
  p.dv = dv;
  p.derase = derase;
  p.dwrite = dwrite;
  p.dg = dg;
  const size_t G = size_t(d.B) * d.N * d.H;
  const bool pc = d.dw == d.K && d.K > 1;
  const bool f32 = grad_dtype == DN_F32;
  // One pass for head_v_dim 64 or 128, else passes of 128 value columns (the
  // last of 64 when head_v_dim is an odd multiple of 64).
  const int passes = d.V <= 128 ? 1 : int((d.V + 127) / 128);
  const size_t rows = size_t(d.B) * d.S * d.H;
  p.vs = int(d.V);
  p.pq = partials;
  p.pk = p.pq ? p.pq + rows * d.K : nullptr;
  p.pe = p.pk ? p.pk + rows * d.K : nullptr;
  p.pg = p.pe ? p.pe + rows * d.ew : nullptr;
  p.pw = p.pg ? p.pg + rows * d.dw : nullptr;
  p.pda = nullptr;
  p.koff = 0;
  if (partials && !pc && d.V > 128) {
    const size_t head = align_up(rows * (2 * d.K + d.ew + d.dw + (d.ww == 1 ? 1 : 0)) *
                                     sizeof(float), 256);
    p.pda = reinterpret_cast<float*>(reinterpret_cast<char*>(partials) + head);
  }
  ProfScope ps("dn_mfma_chunk_bwd", stream);
#define DN_CB(KD, VD, PCV, TG)                                                                  \
  hipLaunchKernelGGL((mfma_chunk_bwd_kernel<KD, VD, PCV, TG>), dim3(unsigned(G)), dim3(kNT), 0, \
                     stream, p)
#define DN_CB_L(KD, VD, TG)                                                                    \
  hipLaunchKernelGGL((mfma_chunk_bwd_kernel<KD, VD, false, TG, true>), dim3(unsigned(G)),       \
                     dim3(kNT), 0, stream, p)
#define DN_CB_LV(KD, TG)                           \
  do {                                             \
    if (vd == 128) DN_CB_L(KD, 128, TG);           \
    else DN_CB_L(KD, 64, TG);                      \
  } while (0)
#define DN_CB_E(KD, TG)                                                                          \
  hipLaunchKernelGGL((mfma_chunk_bwd_kernel<KD, 128, false, TG, false, true>), dim3(unsigned(G)), \
                     dim3(kNT), 0, stream, p)
#define DN_CB_T(KD, VD, PCV)              \
  do {                                    \
    if (f32) DN_CB(KD, VD, PCV, float);   \
    else DN_CB(KD, VD, PCV, bf16);        \
  } while (0)
#define DN_CB_P(KD, VD)                   \
  do {                                    \
    if (pc) DN_CB_T(KD, VD, true);        \
    else DN_CB_T(KD, VD, false);          \
  } while (0)
  if (d.K == 256) {
    // Per value pass, the two key halves; the sums over key channels pass
    // through the partials across all 2·passes launches (rpass).
#define DN_CB2(VD, TG, LP, EP)                                                                   \
  hipLaunchKernelGGL((mfma_chunk_bwd_kernel<128, VD, false, TG, LP, EP, 256>), dim3(unsigned(G)), \
                     dim3(kNT), 0, stream, p)
#define DN_CB2_K(VD, LP, EP)                    \
  do {                                          \
    if (f32) DN_CB2(VD, float, LP, EP);         \
    else DN_CB2(VD, bf16, LP, EP);              \
  } while (0)
    const int launches = 2 * passes;
    for (int i = 0; i < passes; ++i) {
      const int vd = passes == 1 ? int(d.V) : i + 1 < passes || d.V % 128 == 0 ? 128 : 64;
      p.voff = 128 * i;
      p.pass = passes == 1 ? 0 : i == 0 ? 1 : i + 1 == passes ? 3 : 2;
      for (int half = 0; half < 2; ++half) {
        const int j = 2 * i + half;
        p.koff = 128 * half;
        p.rpass = j == 0 ? 1 : j + 1 == launches ? 3 : 2;
        if (p.pass == 3) {
          if (vd == 128) DN_CB2_K(128, true, false); else DN_CB2_K(64, true, false);
        } else if (p.pass != 0) {
          DN_CB2_K(128, false, true);
        } else if (vd == 128) {
          DN_CB2_K(128, false, false);
        } else {
          DN_CB2_K(64, false, false);
        }
        const hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
      }
    }
#undef DN_CB2_K
#undef DN_CB2
    return hipGetLastError();
  }
  for (int i = 0; i < passes; ++i) {
    const int vd = passes == 1 ? int(d.V) : i + 1 < passes || d.V % 128 == 0 ? 128 : 64;
    p.voff = 128 * i;
    p.pass = passes == 1 ? 0 : i == 0 ? 1 : i + 1 == passes ? 3 : 2;
    p.rpass = p.pass;
    if (p.pass == 3 && !pc) {
      if (d.K == 128) {
        if (f32) DN_CB_LV(128, float); else DN_CB_LV(128, bf16);
      } else {
        if (f32) DN_CB_LV(64, float); else DN_CB_LV(64, bf16);
      }
    } else if ((p.pass == 1 || p.pass == 2) && !pc) {
      if (d.K == 128) {
        if (f32) DN_CB_E(128, float); else DN_CB_E(128, bf16);
      } else {
        if (f32) DN_CB_E(64, float); else DN_CB_E(64, bf16);
      }
    } else if (d.K == 128) {
      if (vd == 128) DN_CB_P(128, 128); else DN_CB_P(128, 64);
    } else {
      if (vd == 128) DN_CB_P(64, 128); else DN_CB_P(64, 64);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
#undef DN_CB_P
#undef DN_CB_E
#undef DN_CB_LV
#undef DN_CB_L
#undef DN_CB_T
#undef DN_CB
  return hipGetLastError();
}

}  // namespace dn
