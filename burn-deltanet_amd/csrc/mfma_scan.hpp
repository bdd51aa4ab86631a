// The chunk scan of the two-kernel MFMA forward (bf16 MFMA, fp32 state),
// shared by the translation units that instantiate it: chunk_fwd_mfma.hip
// (the forward, the backward's states scan, the segmented scan) and
// chunk_fwd_norm.hip (the variants with the output norm in the y write).
#pragma once

#include <type_traits>

#include "activations.hpp"
#include "dn_common.hpp"
#include "mfma_util.hpp"

namespace dn {
namespace {

constexpr int kL = 64;  // chunk length

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
  uint16_t* sink;  // one y row: the target of padded tokens' writes
  float* gc;       // [G][64]
  // Per-channel gates (GDN-2) only:
  int ew, ww;      // erase / write gate widths (1 or K / 1 or V); the decay has width K
  uint16_t* Kg;    // [G][64][K] bf16(e⊙e^G⊙K), hi part
  uint16_t* Kglo;  // [G][64][K] its lo part
  uint16_t* Qg;    // [G][64][K] bf16(scale·e^G⊙Q)
  float* egl;      // [G][K] e^{G_last} per key channel
  float* states;   // [G][K][V] fp32 state entering each chunk (states mode of the scan)
  // Segmented scan: the sequence cut into seg_p segments of whole chunks,
  // segment s of batch b scanned as batch b·seg_p + s of a seg_p times
  // shorter sequence (the same token rows and chunk tiles). seg = 0: off;
  // 1: each segment's transition M (the scan of K extra state columns that
  // start at the identity and see no v) and offset H (the end state from
  // S = 0); 2: outputs and states from the carried segment starts.
  int seg, seg_p;
  int vx;           // state columns the launch covers: V, or V + K when seg = 1
  float* seg_m;     // [B·seg_p·H][K][K] M of each segment (seg = 1)
  float* seg_h;     // [B·seg_p·H][K][V] H of each segment (seg = 1)
  float* seg_start; // [B·seg_p·H][K][V] each segment's start state (the carry's output)
  float* seg_final; // [B·H][K][V] the last segments' end states (seg = 2)
  // The output norm fused into the y write (NORM scans): OutNorm::forward
  // (norm.rs:106-144), y / √(mean_v(y²) + ε) · γ [· silu(gate)], per token
  // and head over the head's V columns.
  const void* ng;           // gate rows in y's dtype (NULL: OutNorm::Plain); token row r,
                            // head h at ng + r·ng_stride + h·V
  long long ng_stride;      // below 2^31 / 64 (a chunk's rows at 32-bit offsets)
  const float* nw;          // γ [V]
  float neps;
  // A head's V columns span `ntile` workgroups; each publishes its per-token
  // partial sums of y² for chunk n as 64-bit words (n + 1) << 32 | bits,
  // [launch B·H][ntile][4 slots by chunk][64 tokens], cleared before the
  // launch, and reads its partners' (a cooperative launch keeps the whole
  // grid resident). A wait that reaches nspin polls gives up, counts itself
  // in *nfault and uses 0 for the missing sum.
  unsigned long long* nx;
  int* nfault;
  int nspin;
};

// ---------------------------------------------------------------------------
// scan
// ---------------------------------------------------------------------------
// The staged operand tiles use the permuted contraction index of perm_pos
// (mfma_util.hpp): S, X and V' accumulator tiles feed the MFMAs in place.

// ST (states mode, for the backward's recompute): the fp32 state entering
// each chunk is written to p.states and y is not written. SEG: the
// segmented scan's mode (MfmaParams::seg), 0 for an unsegmented scan.
// x, hidden from the optimiser: the output norm's steps derive their lane
// indices from such a copy of the thread id, so that their addresses are
// recomputed inside each step rather than hoisted out of the chunk loop,
// where they would stay live beside the scan's state and spill.
__device__ inline int scan_opaque(int x) {
  asm volatile("" : "+v"(x));
  return x;
}

// NORM (SEG ≠ 1, not ST): y leaves through OutNorm. Chunk n's y is written
// unnormalised, its per-token partial Σy² over the workgroup's columns goes
// to LDS; at the top of chunk n+1 wave 0 sums the waves' partials and
// publishes them to the head's other column workgroups; after phase 2 of
// chunk n+2 every lane reads its tokens' partner sums (published a chunk and
// a half earlier, so in the steady state nothing waits), re-reads its own y
// values of chunk n and the gate, and after phase 3 writes the normalised
// output over them. The last two chunks finish after the loop.
// NORM: 0 none, 1 OutNorm::Plain, 2 OutNorm::Gated with the gate in y's dtype.
// G4 (ST): the states in row groups of four ([G][K/4][V][4], states_g4).
template <int K, class TY, int WAVES, bool PC, bool ST = false, int SEG = 0, int NORM = 0,
          bool G4 = false>
__global__ __launch_bounds__(64 * WAVES) void mfma_scan_kernel(MfmaParams p) {
  static_assert(NORM == 0 || (!ST && SEG != 1), "the output norm applies to y");
  constexpr int KK = K / 32;      // 32-deep k-steps over the key axis
  constexpr int RBK = K / 16;     // 16-row blocks of the state
  constexpr int NT = 64 * WAVES;
  constexpr int BW = 16 * WAVES;  // value columns per workgroup
  // One chunk's operand tiles (bf16 elements): K, Q [64][K] (per-channel
  // gates: kg hi, qg and kg lo instead); T, Tlo, attn [64][64]; per-channel
  // gates only: Kcᵀ [K][64]. With per-head gates the state update reads Kᵀ
  // from the K tile through the LDS transpose read and puts the factor
  // e^{G_last−G} on V' (Kcᵀ·V' = Kᵀ·(e^{G_last−G}⊙V')), which saves Kcᵀ's
  // round trip through HBM.
  // Double-buffered for per-head gates: the next chunk is staged while this
  // one is consumed, so one barrier per chunk suffices. The per-channel
  // tiles with y, and head_k_dim 256's (88 KB a chunk), do not fit twice in
  // LDS: they are staged between two barriers. (Without y the per-channel
  // tiles take 64 KB; double-buffered, config 5's two-wave states scan ran
  // slower, 861 → 1057 µs.) (A head_k_dim 256 variant that
  // kept the K and [64][64] tiles double-buffered and restaged a single Q
  // tile after a barrier behind phase 1 measured slower, 487 → 652 µs at
  // B=8 T=4096 H=16 dv=256: its extra staging registers spill in the loop.)
  // Without y (the states mode, the transition pass) neither Q (qg) nor attn
  // is staged: they only form y.
  constexpr bool kYOut = !ST && SEG != 1;              // y is written
  constexpr int NKQ = 1 + (kYOut ? 1 : 0) + (PC ? 1 : 0);  // K-wide tiles: K (, Q) (, kg lo)
  constexpr int NLL = kYOut ? 3 : 2;                   // [64][64] tiles: T, Tlo (, attn)
  constexpr int oK = 0, oQ = oK + kL * K, oKl = (kYOut ? 2 : 1) * kL * K, oT = NKQ * kL * K,
                oTl = oT + kL * kL, oAt = oTl + kL * kL, oKc = oT + NLL * kL * kL,
                BUF = NKQ * kL * K + NLL * kL * kL + (PC ? K * kL : 0);
  constexpr int C16 = BUF / 8;    // 16-byte chunks per chunk's tiles
  // The forward with per-head gates (not the states mode) reads T, T lo and
  // attn packed, kTriTrio elements per chunk-head from p.T (mfma_util.hpp);
  // a packed round's last lanes may idle, in whole waves.
  constexpr bool kCT = !PC && tri_packed(K, ST);
  constexpr int NKQC = NKQ * kL * K / 8;           // 16-byte chunks of the K-wide tiles
  constexpr int NCT = NLL * kTriPacked / 8;        // of the packed [64][64] tiles
  static_assert(NKQC % NT == 0 && NCT % 64 == 0, "staging rounds");
  static_assert(kCT || C16 % NT == 0, "staging assumes whole rounds");
  constexpr int NRC = kCT ? (NCT + NT - 1) / NT : 1;  // packed rounds
  constexpr int NPF = kCT ? NKQC / NT + NRC : C16 / NT;  // chunks staged per lane
  constexpr int NBUF = PC || K > 128 ? 1 : 2;
  __shared__ __attribute__((aligned(16))) uint16_t tiles[NBUF][BUF];
  __shared__ float gxe[NBUF][kL], gwr[NBUF][kL], gys[NBUF][kL], gegl[NBUF];
  // e^{G_last−G} per token (per-head gates), rows of V' for the state update.
  __shared__ __attribute__((aligned(16))) float gkc[PC ? 1 : NBUF][kL];
  __shared__ float gch[PC ? K : 1];  // e^{G_last} per key channel (per-channel gates)
  // NORM: per-wave partial Σy² of chunk n [n & 1][token][wave] (pitch
  // WAVES + 1), and the workgroup's sum per token [n & 1][token].
  constexpr bool kNorm = NORM != 0;
  __shared__ float nsq[kNorm ? 2 : 1][kNorm ? kL : 1][kNorm ? WAVES + 1 : 1];
  __shared__ float nown[kNorm ? 2 : 1][kNorm ? kL : 1];
  __shared__ float nrsl[kNorm ? 2 : 1][kNorm ? kL : 1];  // 1/√(mean + ε) per token
  __shared__ __attribute__((aligned(16))) float ngam[kNorm ? BW : 1];  // γ of the columns

  const int ntile = (SEG == 1 ? p.vx : p.V) / BW;
  const int BH = p.B * p.H;
  // XCD-aware: the `ntile` workgroups of one (b, h) get ids ≡ (mod 8).
  const int id = blockIdx.x;
  const int group = id / (8 * ntile), within = id % (8 * ntile);
  const int tile = within / 8, bh = group * 8 + within % 8;
  if (bh >= BH) return;
  const int b = bh / p.H, h = bh % p.H;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int r16 = lane & 15, q4 = lane >> 4, k8 = 8 * q4;
  const int jw = tile * BW + 16 * wave;  // this wave's first value column
  const int jl = jw + r16;               // this lane's column (accumulator layout)
  // A transition column (seg = 1): column jl − V of the identity, no v input.
  const bool trans = SEG == 1 && jw >= p.V;

  // S[:, jw…jw+15] in accumulator layout: RBK row blocks of 16.
  f32x4 S[RBK];
  if constexpr (SEG == 1) {
#pragma unroll
    for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r)
        S[rb][r] = trans && 16 * rb + 4 * q4 + r == jl - p.V ? 1.f : 0.f;
  } else {
    const float* sin = p.s_in + size_t(bh) * K * p.V + jl;
#pragma unroll
    for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[rb][r] = sin[size_t(16 * rb + 4 * q4 + r) * p.V];
  }

  const size_t tokstride = size_t(p.H);  // rows between consecutive tokens
  const size_t bh_row0 = size_t(b) * p.S * p.H + h;
  auto chunk_of = [&](int n) { return (size_t(b) * p.N + n) * p.H + h; };

  // Staging. Global reads use a wave-uniform base (per chunk) plus a 32-bit
  // lane offset, and are unconditional: rows past the sequence end are
  // clamped to its last row (their gates are zero, so those values only ever
  // meet zero factors), which keeps every iteration's memory operations
  // identical and the compiler's in-order vmcnt waits exact.
  const int HK = p.H * K;
  const uint32_t kcol = uint32_t(8 * (tid % (K / 8)));
  const uint32_t koff = uint32_t((tid / (K / 8)) * HK) + kcol;
  uint4 pf[NPF];
  float pgc, pgl, per, pwr, pch;
  auto ld16 = [](const uint16_t* base, uint32_t elems) {
    return *reinterpret_cast<const uint4*>(reinterpret_cast<const char*>(base) + 2u * elems);
  };
  // fetch / stage cover rounds m0 … m1−1 of the staging, the gates with
  // round 0 (every call passes constants).
  auto fetch = [&](int n, int m0, int m1) {
    const size_t cid = chunk_of(n);
    const int rl = min(kL, p.S - n * kL);  // valid rows of this chunk (≥ 1)
    const size_t row0 = bh_row0 + size_t(n) * kL * tokstride;
#pragma unroll
    for (int m = 0; m < NPF; ++m) {
      if (m < m0 || m >= m1) continue;
      // The tile boundaries are multiples of NT, so the kind of chunk
      // tid + NT·m depends on m only (a constant once the loop is unrolled).
      const int i0 = NT * m;
      if (i0 < NKQ * kL * K / 8) {
        const int which = i0 / (kL * K / 8);
        if constexpr (PC) {
          // kg, qg and kg lo: written by the intra kernel per chunk-head
          // (zero past the sequence end).
          const uint16_t* base = which == 0 ? p.Kg : (kYOut && which == 1) ? p.Qg : p.Kglo;
          pf[m] = ld16(base + cid * kL * K + 8 * (i0 - which * (kL * K / 8)), 8u * tid);
        } else {
          // Row tid/(K/8) + rowc, clamped through its (monotonic) offset.
          const uint32_t rowc = uint32_t((i0 - which * (kL * K / 8)) / (K / 8));
          const uint32_t klast = uint32_t((rl - 1) * HK) + kcol;
          pf[m] = ld16((which ? p.q : p.k) + row0 * K, min(koff + rowc * uint32_t(HK), klast));
        }
      } else if constexpr (kCT) {
        const int cc0 = i0 - NKQC;  // the round's first packed chunk
        if (cc0 + NT <= NCT || tid < NCT - cc0)
          pf[m] = ld16(p.T + cid * kTriTrio, 8u * uint32_t(cc0 + tid));
      } else if (i0 < (NKQ * kL * K + NLL * kL * kL) / 8) {
        const int ii0 = i0 - NKQ * kL * K / 8;
        const int which = ii0 / (kL * kL / 8);
        const uint16_t* base = which == 0 ? p.T : which == 1 ? p.Tlo : p.attn;
        pf[m] = ld16(base + cid * kL * kL + 8 * (ii0 - which * (kL * kL / 8)), 8u * tid);
      } else {
        const int e0 = i0 - (NKQ * kL * K + NLL * kL * kL) / 8;
        pf[m] = ld16(p.KcT + cid * K * kL + 8 * e0, 8u * tid);
      }
    }
    if (m0 > 0) return;
    if constexpr (PC) {
      pch = p.egl[cid * K + (tid % K)];
    } else {
      const int lc = min(lane, rl - 1);
      pgc = p.gc[cid * kL + lane];
      pgl = p.gc[cid * kL + kL - 1];
      const float e = p.erase[row0 + size_t(lc) * tokstride];
      const float w = p.write[row0 + size_t(lc) * tokstride];
      per = lane < rl ? e : 0.f;
      pwr = lane < rl ? w : 0.f;
    }
  };
  // Staging addresses are loop invariant: lane tid writes the halves of
  // 16-byte chunk (row r, column group c) of every tile, rows advancing by a
  // multiple of 8 per round m (which flips the K-wide swizzle by m-constant
  // bits only).
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
  // Packed chunk NT·j + tid: tile `which`, block st (rows 16·tril_tb(st) …,
  // columns 32·tril_kk(st) …), row r and column group cg inside it.
  int cb0[NRC], cb1[NRC];
  if constexpr (kCT) {
#pragma unroll
    for (int j = 0; j < NRC; ++j) {
      const int cc = NT * j + tid;
      const int which = cc / (kTriPacked / 8), ci = cc % (kTriPacked / 8);
      const int st = ci >> 6, r = (ci >> 2) & 15, cg = ci & 3;
      const int row = 16 * tril_tb(st) + r, col = 32 * tril_kk(st) + 8 * cg;
      const int base = which == 0 ? oT : which == 1 ? oTl : oAt;
      cb0[j] = base + tile_at<kL>(row, perm_pos(col));
      cb1[j] = base + tile_at<kL>(row, perm_pos(col + 4));
    }
  }
  auto stage = [&](int buf, int m0, int m1) {
    uint16_t* tl = tiles[buf];
#pragma unroll
    for (int m = 0; m < NPF; ++m) {
      if (m < m0 || m >= m1) continue;
      const int i0 = NT * m;
      int b0, b1;
      if (i0 < NKQ * kL * K / 8) {
        const int which = i0 / (kL * K / 8);
        const int dr = (i0 - which * (kL * K / 8)) / KC8;  // row advance, a multiple of 8
        const int base = (which == 0 ? oK : (kYOut && which == 1) ? oQ : oKl) + dr * K;
        const bool flip = K >= 128 && (dr & 8);
        b0 = base + (flip ? aK0x : aK0);
        b1 = base + (flip ? aK1x : aK1);
      } else if constexpr (kCT) {
        const int cc0 = i0 - NKQC;
        if (!(cc0 + NT <= NCT || tid < NCT - cc0)) continue;
        b0 = cb0[cc0 / NT];
        b1 = cb1[cc0 / NT];
      } else if (i0 < (NKQ * kL * K + NLL * kL * kL) / 8) {
        const int ii0 = i0 - NKQ * kL * K / 8;
        const int which = ii0 / (kL * kL / 8), dr = (ii0 - which * (kL * kL / 8)) / LC8;
        const int base = (which == 0 ? oT : which == 1 ? oTl : oAt) + dr * kL;
        b0 = base + a60;
        b1 = base + a61;
      } else {
        const int dr = (i0 - (NKQ * kL * K + NLL * kL * kL) / 8) / LC8;
        b0 = oKc + dr * kL + a60;
        b1 = oKc + dr * kL + a61;
      }
      *reinterpret_cast<uint2*>(&tl[b0]) = make_uint2(pf[m].x, pf[m].y);
      *reinterpret_cast<uint2*>(&tl[b1]) = make_uint2(pf[m].z, pf[m].w);
    }
    if (m0 > 0) return;
    if constexpr (PC) {
      if (tid < K) gch[tid] = pch;
    } else if (wave == 0) {
      const float eg = __expf(pgc);
      gxe[buf][lane] = per * eg;
      gwr[buf][lane] = pwr;
      gys[buf][lane] = p.scale * eg;
      gkc[buf][lane] = __expf(pgl - pgc);
      if (lane == 0) gegl[buf] = __expf(pgl);
    }
  };
  // v[t][jl] for this lane's 16 tokens (4 row blocks × 4), as bf16 pairs.
  // Offsets grow with the token, so clamping the token to the chunk's last
  // row is clamping the offset: min(t·HV + jl, (rl−1)·HV + jl), where
  // t·HV + jl = vlane + (16·tb + r)·HV with a per-lane vlane.
  uint32_t vA[4][2];
  const int HV = p.H * p.V;
  // A transition column reads column jl − V (< K ≤ V) and weighs it by zero:
  // no branch around the loads, whose registers would be copied, and waited
  // for, where the branches join.
  const int jv = trans ? jl - p.V : jl;
  const uint32_t vlane = uint32_t(4 * q4 * HV + jv);
  auto load_v = [&](int n) {
    const int rl = min(kL, p.S - n * kL);
    const uint16_t* vb = p.v + (bh_row0 + size_t(n) * kL * tokstride) * p.V;
    const uint32_t vlast = uint32_t((rl - 1) * HV) + uint32_t(jv);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int r2 = 0; r2 < 2; ++r2) {
        const uint32_t t0 = uint32_t(16 * tb + 2 * r2);
        const uint32_t o0 = min(vlane + t0 * uint32_t(HV), vlast);
        const uint32_t o1 = min(vlane + (t0 + 1) * uint32_t(HV), vlast);
        const uint32_t x0 = *reinterpret_cast<const uint16_t*>(
            reinterpret_cast<const char*>(vb) + 2u * o0);
        const uint32_t x1 = *reinterpret_cast<const uint16_t*>(
            reinterpret_cast<const char*>(vb) + 2u * o1);
        vA[tb][r2] = x0 | (x1 << 16);
      }
  };
  // Per-channel gates: the write gate w[t][jl] for the same 16 tokens (width
  // V, or one value per token); zero past the sequence end.
  float wA[4][4];
  auto load_w = [&](int n) {
    if constexpr (PC) {
      const int rl = min(kL, p.S - n * kL);
      const float* wb = p.write + (bh_row0 + size_t(n) * kL * tokstride) * p.ww +
                        (p.ww == 1 ? 0 : jv);
      const int hw = p.H * p.ww;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = 16 * tb + 4 * q4 + r;
          const float w = wb[size_t(min(t, rl - 1)) * hw];
          wA[tb][r] = t < rl ? w : 0.f;
        }
    }
  };
  auto as8 = [](const uint4& x) { return __builtin_bit_cast(bf16x8, x); };

  // --- NORM: the output norm over the head's V columns ---------------------
  // Lane (r16, q4) holds value columns jw + 4q4 … +3 of token 16tb + r16 in
  // yt[tb]. Per chunk n, across the chunk steps that follow it:
  //   end of n        each wave's partial Σy² per token → nsq[n & 1]
  //   top of n+1      wave 0: the workgroup's sums → nown, published
  //   n+2, phase 3    wave 0: the partners' sums of chunk n loaded
  //   end of n+2      wave 0: their tags checked (waiting only if one is
  //                   late), 1/√(mean + ε) per token → nrs; every lane
  //                   loads its y values of chunk n (written unnormalised)
  //                   and the gate
  //   top of n+3      every lane stores the normalised output, before the
  //                   chunk's own loads: the values wait across the barrier,
  //                   where few registers are live.
  constexpr int kNormPre = 1;  // partner words prefetched a chunk ahead
  auto norm_partial = [&](int n, const f32x4* yv) {
    if constexpr (kNorm) {
      const int lane = scan_opaque(tid) & 63, q4 = lane >> 4;
      float ps[4];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        float x = yv[tb][0] * yv[tb][0];
#pragma unroll
        for (int r = 1; r < 4; ++r) x = fmaf(yv[tb][r], yv[tb][r], x);
        x += __shfl_xor(x, 16, 64);
        x += __shfl_xor(x, 32, 64);
        ps[tb] = x;
      }
      // lane 16·q4 + r16 keeps token 16·q4 + r16, i.e. token = lane
      const float mine = q4 == 0 ? ps[0] : q4 == 1 ? ps[1] : q4 == 2 ? ps[2] : ps[3];
      nsq[n & 1][lane][wave] = mine;
    }
  };
  auto nslot = [&](int n, int j) {
    return p.nx + ((size_t(bh) * ntile + j) * 4 + (n & 3)) * kL + (scan_opaque(tid) & 63);
  };
  auto norm_publish = [&](int n) {
    if constexpr (kNorm) {
      if (wave == 0) {
        const int lane = scan_opaque(tid) & 63;
        float sum = 0.f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) sum += nsq[n & 1][lane][w];
        nown[n & 1][lane] = sum;
        if (ntile > 1)
          __hip_atomic_store(nslot(n, tile),
                             (static_cast<unsigned long long>(n + 1) << 32) | __float_as_uint(sum),
                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
    }
  };
  unsigned long long npre[kNormPre];
  auto norm_fetch = [&](int n) {
    if constexpr (kNorm) {
      if (wave == 0) {
#pragma unroll
        for (int i = 0; i < kNormPre; ++i) {
          const int j = i < tile ? i : i + 1;  // the i-th partner
          npre[i] = j < ntile ? __hip_atomic_load(nslot(n, j), __ATOMIC_RELAXED,
                                                  __HIP_MEMORY_SCOPE_AGENT)
                              : 0ull;
        }
      }
    }
  };
  // Wave 0: chunk n's per-token sums complete; prefetched: npre holds the
  // first partners' words (else they are loaded here).
  auto norm_gather = [&](int n, bool prefetched) {
    if constexpr (kNorm) {
      if (wave == 0) {
        const int lane = scan_opaque(tid) & 63;
        const unsigned long long want = static_cast<unsigned long long>(n + 1);
        float tot = nown[n & 1][lane];
        for (int j = 0, i = 0; j < ntile; ++j) {
          if (j == tile) continue;
          unsigned long long w = (prefetched && i < kNormPre)
                                     ? npre[i]
                                     : __hip_atomic_load(nslot(n, j), __ATOMIC_RELAXED,
                                                         __HIP_MEMORY_SCOPE_AGENT);
          ++i;
          for (int it = 0; (w >> 32) != want; ++it) {
            if (it >= p.nspin) {
              atomicAdd(p.nfault, 1);
              w = want << 32;
              break;
            }
            __builtin_amdgcn_s_sleep(2);
            w = __hip_atomic_load(nslot(n, j), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
          }
          tot += __uint_as_float(uint32_t(w));
        }
        nrsl[n & 1][lane] = rsqrtf(tot * (1.0f / float(p.V)) + p.neps);
      }
    }
  };
  // Every lane: its y and gate values of chunk n, from the chunk's first
  // row (a wave-uniform base) at 32-bit offsets (token rows are 32-bit
  // addressable, token_rows_fit_32bit; the gate's stride is checked by the
  // caller). Rows past the sequence end clamped to its last row (nothing is
  // stored there). Unconditional loads: a load under a condition would make
  // its first use wait for every load in flight.
  using YW = std::conditional_t<sizeof(TY) == 2, uint2, uint4>;  // 4 values of y or gate
  YW nyv[4], ngv[NORM == 2 ? 4 : 1];
  auto norm_rows = [&](int n) { return size_t(b) * p.S + size_t(n) * kL; };
  auto norm_start = [&](int n) {
    if constexpr (kNorm) {
      const int lane = scan_opaque(tid) & 63, r16 = lane & 15, q4 = lane >> 4;
      const uint32_t col = uint32_t(16 * wave + 4 * q4);
      const int rl = min(kL, p.S - n * kL);
      const size_t row0 = norm_rows(n);
      const char* yb = reinterpret_cast<const char*>(static_cast<const TY*>(p.y) +
                                                     (row0 * p.H + h) * size_t(p.V) + tile * BW);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const uint32_t t = uint32_t(min(16 * tb + r16, rl - 1));
        nyv[tb] = *reinterpret_cast<const YW*>(yb + sizeof(TY) * (t * uint32_t(HV) + col));
      }
      if constexpr (NORM == 2) {
        const char* gb = reinterpret_cast<const char*>(
            static_cast<const TY*>(p.ng) + row0 * size_t(p.ng_stride) + size_t(h) * p.V +
            tile * BW);
#pragma unroll
        for (int tb = 0; tb < 4; ++tb) {
          const uint32_t t = uint32_t(min(16 * tb + r16, rl - 1));
          ngv[tb] = *reinterpret_cast<const YW*>(
              gb + sizeof(TY) * (t * uint32_t(p.ng_stride) + col));
        }
      }
    }
  };
  auto unpack4 = [](const YW& w, float* f) {
    if constexpr (sizeof(TY) == 2) {
      f[0] = lo_f(w.x);
      f[1] = hi_f(w.x);
      f[2] = lo_f(w.y);
      f[3] = hi_f(w.y);
    } else {
      f[0] = __uint_as_float(w.x);
      f[1] = __uint_as_float(w.y);
      f[2] = __uint_as_float(w.z);
      f[3] = __uint_as_float(w.w);
    }
  };
  // The normalised output of chunk n over its unnormalised y (after a
  // barrier that follows norm_gather(n)).
  auto norm_finish = [&](int n) {
    if constexpr (kNorm) {
      const int lane = scan_opaque(tid) & 63, r16 = lane & 15, q4 = lane >> 4;
      const uint32_t col = uint32_t(16 * wave + 4 * q4);
      const int rl = min(kL, p.S - n * kL);
      const float4 gw = *reinterpret_cast<const float4*>(&ngam[col]);
      const float gam[4] = {gw.x, gw.y, gw.z, gw.w};
      char* yb = reinterpret_cast<char*>(static_cast<TY*>(p.y) +
                                         (norm_rows(n) * p.H + h) * size_t(p.V) + tile * BW);
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int t = 16 * tb + r16;
        const float rs = nrsl[n & 1][t];
        float yv[4], o[4];
        unpack4(nyv[tb], yv);
        if constexpr (NORM == 2) {
          float gv[4];
          unpack4(ngv[tb], gv);
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = yv[r] * rs * gam[r] * (gv[r] * sigmoidf_(gv[r]));
        } else {
#pragma unroll
          for (int r = 0; r < 4; ++r) o[r] = yv[r] * rs * gam[r];
        }
        if (t < rl) {
          char* dst = yb + sizeof(TY) * (uint32_t(t) * uint32_t(HV) + col);
          if constexpr (sizeof(TY) == 2)
            *reinterpret_cast<uint2*>(dst) = make_uint2(pk_bf16(o[0], o[1]), pk_bf16(o[2], o[3]));
          else
            *reinterpret_cast<float4*>(dst) = make_float4(o[0], o[1], o[2], o[3]);
        }
      }
    }
  };
  if constexpr (kNorm) {
    // γ of this workgroup's columns, read once.
    if (tid < BW) ngam[tid] = p.nw[tile * BW + tid];
  }

  fetch(0, 0, NPF);
  load_v(0);
  load_w(0);
  stage(0, 0, NPF);
  __syncthreads();
  for (int n = 0; n < p.N; ++n) {
    const int cur = NBUF == 1 ? 0 : (n & 1);
    const int nn = n + 1 < p.N ? n + 1 : n;  // the last chunk prefetches itself again
    const uint16_t* tl = tiles[cur];
    const float egl = PC ? 1.f : gegl[cur];
    // The next chunk's tiles are fetched at the top, so the loads have all
    // three phases to land before stage() writes them to LDS (config 2 scan
    // 392 → 376 µs, config 5's per-channel scan 1165 → 870 µs). The
    // per-channel states mode (the backward's recompute) measured slower so
    // (1055 → 1105 µs): its fetch stays after phase 1.
    constexpr bool kFetchTop = !(PC && ST);
    // Eight-wave double-buffered scans: the next chunk's tiles in two
    // halves, the first staged after phase 1 (the other buffer is free all
    // chunk), which halves the registers holding them (config 2 scan 339 →
    // 312 µs). The two-wave scan (36 rounds per lane) and the states mode
    // measured slower so (config 4 1.09 → 1.24 ms).
    constexpr bool kHalf = NBUF == 2 && WAVES == 8 && !ST;
    constexpr int NH = kHalf ? (NPF + 1) / 2 : NPF;
    if constexpr (kFetchTop) fetch(nn, 0, NH);
    // The output norm of chunk n − 3 once this chunk's tile loads are in
    // flight (its wait is for older loads only).
    if (n >= 3) norm_finish(n - 3);
    if (n >= 1) norm_publish(n - 1);
    if constexpr (ST && G4) {
      // a lane's four rows of its column as one 16-byte store
      float4* sdst = reinterpret_cast<float4*>(p.states + chunk_of(n) * K * p.V) + jl;
#pragma unroll
      for (int rb = 0; rb < RBK; ++rb)
        sdst[size_t(4 * rb + q4) * p.V] = make_float4(S[rb][0], S[rb][1], S[rb][2], S[rb][3]);
    } else if constexpr (ST) {
      float* sdst = p.states + chunk_of(n) * K * p.V + jl;
#pragma unroll
      for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) sdst[size_t(16 * rb + 4 * q4 + r) * p.V] = S[rb][r];
    }

    // Phase 1: X = w⊙V − (e⊙e^G)⊙(K·S) in [token][column] orientation, and
    // yᵀ = Sᵀ·Qᵀ in [column][token] orientation. The S fragments (hi, lo) of
    // k-step kk are the B operand of K·S and the A operand of Sᵀ·Qᵀ (same
    // lane layout). Fragment reads run one (kk, tb) step ahead of the MFMAs.
    // Two-wave per-head scans (one wave per SIMD) interleave VALU work with
    // independent MFMAs by hand: in phase 1 the next k-step's S fragments
    // are split while this one's MFMAs run, one MFMA to two VALU
    // instructions (config 4 1.09 → 1.05 ms). With two waves per SIMD the
    // other wave covers the split, and so interleaved the eight-wave scan
    // measured slower (315 → 345 µs), as did the per-channel states mode;
    // S's gate products placed under phase 3's attn MFMAs likewise (config 4
    // 1.05 → 1.20 ms), and X's second k-step split under phase 2's first
    // nine MFMAs (1.05 → 1.14 ms).
    constexpr bool kPipe = WAVES == 2 && !PC && !ST;
    f32x4 X[4], yt[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
      X[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
      yt[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }
    {
      // Fragment reads run PD steps ahead of the MFMAs (a ring of PD + 1).
      constexpr int PD = 2, NR = PD + 1, NSTEP = 4 * KK;
      bf16x8 kf[NR], qf[NR], kl[NR];
      auto rd = [&](int st) {
        const int at = tile_at<K>(16 * (st & 3) + r16, 32 * (st >> 2) + k8);
        kf[st % NR] = ld8(&tl[oK + at]);
        if constexpr (kYOut) qf[st % NR] = ld8(&tl[oQ + at]);
        if constexpr (PC) kl[st % NR] = ld8(&tl[oKl + at]);
      };
#pragma unroll
      for (int st = 0; st < PD; ++st) rd(st);
      if constexpr (kPipe) {
        uint4 sh = frag_hi(S[0], S[1]);
        uint4 sl = frag_lo(S[0], S[1], sh);
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          uint4 shn = sh, sln = sl;
          if (kk + 1 < KK) {
            shn = frag_hi(S[2 * kk + 2], S[2 * kk + 3]);
            sln = frag_lo(S[2 * kk + 2], S[2 * kk + 3], shn);
          }
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            const int step = 4 * kk + tb;
            if (step + PD < NSTEP) rd(step + PD);
            const int c = step % NR;
            X[tb] = mfma16(kf[c], as8(sh), X[tb]);
            X[tb] = mfma16(kf[c], as8(sl), X[tb]);
            if constexpr (kYOut) yt[tb] = mfma16(as8(sh), qf[c], yt[tb]);
          }
          if (kk + 1 < KK) {
#pragma unroll
            for (int i = 0; i < 12; ++i) {
              __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
              __builtin_amdgcn_sched_group_barrier(0x002, 2, 0);  // two VALU
            }
          }
          sh = shn;
          sl = sln;
        }
      } else {
#pragma unroll
        for (int kk = 0; kk < KK; ++kk) {
          const uint4 sh = frag_hi(S[2 * kk], S[2 * kk + 1]);
          const uint4 sl = frag_lo(S[2 * kk], S[2 * kk + 1], sh);
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            const int step = 4 * kk + tb;
            if (step + PD < NSTEP) rd(step + PD);
            const int c = step % NR;
            X[tb] = mfma16(kf[c], as8(sh), X[tb]);
            X[tb] = mfma16(kf[c], as8(sl), X[tb]);
            // kg carries the fp32 gate factors, so it has a lo part too.
            if constexpr (PC) X[tb] = mfma16(kl[c], as8(sh), X[tb]);
            if constexpr (kYOut) yt[tb] = mfma16(as8(sh), qf[c], yt[tb]);
          }
        }
      }
    }
    if constexpr (!kFetchTop) fetch(nn, 0, NPF);
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int t = 16 * tb + 4 * q4 + r;
        const float vv = (r & 1) ? hi_f(vA[tb][r >> 1]) : lo_f(vA[tb][r >> 1]);
        // Per-channel gates: e⊙e^G is inside kg, scale·e^G inside qg.
        const float wv = trans ? 0.f : (PC ? wA[tb][r] : gwr[cur][t]);
        X[tb][r] = PC ? wv * vv - X[tb][r] : wv * vv - gxe[cur][t] * X[tb][r];
      }
      if constexpr (!PC) {
        const float ysc = gys[cur][16 * tb + r16];
#pragma unroll
        for (int r = 0; r < 4; ++r) yt[tb][r] *= ysc;
      }
    }
    load_v(nn);
    load_w(nn);
    if constexpr (kHalf) {
      stage(cur ^ 1, 0, NH);
      fetch(nn, NH, NPF);
    }

    // Phase 2: V' = T·X with hi + lo parts of both factors (for a chunk of
    // near-identical keys T differences near-equal rows of X).
    uint4 xh[2], xl[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) {
      xh[kk] = frag_hi(X[2 * kk], X[2 * kk + 1]);
      xl[kk] = frag_lo(X[2 * kk], X[2 * kk + 1], xh[kk]);
    }
    f32x4 Vp[4];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb) Vp[tb] = f32x4{0.f, 0.f, 0.f, 0.f};
    {
      // T is lower triangular: its six nonzero (row block, k-step) pairs.
      auto at = [&](int st) { return tile_at<kL>(16 * tril_tb(st) + r16, 32 * tril_kk(st) + k8); };
      bf16x8 th[2], tlo[2];
      th[0] = ld8(&tl[oT + at(0)]);
      tlo[0] = ld8(&tl[oTl + at(0)]);
#pragma unroll
      for (int st = 0; st < kTriSteps; ++st) {
        if (st + 1 < kTriSteps) {
          th[(st + 1) & 1] = ld8(&tl[oT + at(st + 1)]);
          tlo[(st + 1) & 1] = ld8(&tl[oTl + at(st + 1)]);
        }
        const int tb = tril_tb(st), kk = tril_kk(st);
        Vp[tb] = mfma16(th[st & 1], as8(xh[kk]), Vp[tb]);
        Vp[tb] = mfma16(tlo[st & 1], as8(xh[kk]), Vp[tb]);
        Vp[tb] = mfma16(th[st & 1], as8(xl[kk]), Vp[tb]);
      }
    }


    if (n >= 2) norm_fetch(n - 2);
    // Phase 3: yᵀ += V'ᵀ·attnᵀ and S ← e^{G_last}⊙S + (e^{G_last−G}⊙K)ᵀ·V';
    // the bf16 V' fragment is the A operand of the first and the B operand
    // of the second.
    uint4 vf[2], vc[2];
#pragma unroll
    for (int kk = 0; kk < 2; ++kk) vf[kk] = frag_hi(Vp[2 * kk], Vp[2 * kk + 1]);
    if constexpr (!PC) {
      // e^{G_last−G}⊙V': lane (r16, q4) holds rows 16tb + 4q4 … +3 of Vp[tb].
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const float4 c = *reinterpret_cast<const float4*>(&gkc[cur][16 * tb + 4 * q4]);
        Vp[tb][0] *= c.x;
        Vp[tb][1] *= c.y;
        Vp[tb][2] *= c.z;
        Vp[tb][3] *= c.w;
      }
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) vc[kk] = frag_hi(Vp[2 * kk], Vp[2 * kk + 1]);
    }
    {
      // The six nonzero steps of the lower-triangular attn (when y is
      // written), then 2·RBK state update steps, reads one step ahead.
      constexpr int NA = kYOut ? kTriSteps : 0, NS = NA + 2 * RBK;
      auto addr = [&](int st) {
        return st < NA ? oAt + tile_at<kL>(16 * tril_tb(st) + r16, 32 * tril_kk(st) + k8)
                       : oKc + tile_at<kL>(16 * ((st - NA) >> 1) + r16, 32 * ((st - NA) & 1) + k8);
      };
      // Kᵀ's fragment of state rows 16rb … +15 and k-step kk (tokens 32kk …
      // +31 in the permuted order) from the K tile: ds_read_b64_tr_b16 gives
      // lane i of each 16-lane group element i of the 4×4 block that lanes
      // 4j … 4j+3 of the group supply (lane 4j + m: 4 consecutive
      // elements), as its element j. Lane (r16, q4) supplies channels
      // 16rb + 4(r16 & 3) … +3 of token 32kk + 4q4 + (r16 >> 2), and of the
      // token 16 further for the second half, so lane (r16, q4) receives
      // channel 16rb + r16 of tokens 32kk + 4q4 … +3 and 32kk + 16 + 4q4 … +3:
      // operand positions 8q4 … 8q4+7 of the permuted order.
      auto kt_frag = [&](int rb, int kk) {
        const int t = 32 * kk + 4 * q4 + (r16 >> 2);
        const int pos = 32 * (rb >> 1) + 8 * (r16 & 3) + 4 * (rb & 1);
        typedef short v4s __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) v4s lds_v4s;
        const v4s a = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4s*)(&tl[oK + tile_at<K>(t, pos)]));
        const v4s b = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
            (lds_v4s*)(&tl[oK + tile_at<K>(t + 16, pos)]));
        const uint2 ua = __builtin_bit_cast(uint2, a), ub = __builtin_bit_cast(uint2, b);
        return __builtin_bit_cast(bf16x8, make_uint4(ua.x, ua.y, ub.x, ub.y));
      };
      auto frag = [&](int st) {
        if constexpr (!PC)
          if (st >= NA) return kt_frag((st - NA) >> 1, (st - NA) & 1);
        return ld8(&tl[addr(st)]);
      };
      bf16x8 fr[2];
      fr[0] = frag(0);
#pragma unroll
      for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
        for (int r = 0; r < 4; ++r) S[rb][r] *= PC ? gch[16 * rb + 4 * q4 + r] : egl;
#pragma unroll
      for (int st = 0; st < NS; ++st) {
        if (st + 1 < NS) fr[(st + 1) & 1] = frag(st + 1);
        if (st < NA)
          yt[tril_tb(st)] = mfma16(as8(vf[tril_kk(st)]), fr[st & 1], yt[tril_tb(st)]);
        else
          S[(st - NA) >> 1] =
              mfma16(fr[st & 1], as8(PC ? vf[(st - NA) & 1] : vc[(st - NA) & 1]), S[(st - NA) >> 1]);
      }
    }
    // The norm's loads before this chunk's y stores: the wait for them at
    // the top of the next chunk then leaves those stores in flight (stores
    // count in the same in-order counter).
    if (n >= 2) norm_start(n - 2);
    // y: lane (r16, q4) holds columns jw + 4q4 … +3 of token 16tb + r16;
    // rows past the sequence end go to the sink row.
    if constexpr (!ST && SEG != 1) {
      TY* yb = static_cast<TY*>(p.y) + (bh_row0 + size_t(n) * kL * tokstride) * p.V;
      const int rl = p.S - n * kL;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const int t = 16 * tb + r16;
        TY* dst = t < rl ? reinterpret_cast<TY*>(reinterpret_cast<char*>(yb) +
                                                 sizeof(TY) * uint32_t(t * HV + jw + 4 * q4))
                         : reinterpret_cast<TY*>(p.sink) + jw + 4 * q4;
        if constexpr (sizeof(TY) == 2)
          *reinterpret_cast<uint2*>(dst) =
              make_uint2(pk_bf16(yt[tb][0], yt[tb][1]), pk_bf16(yt[tb][2], yt[tb][3]));
        else
          *reinterpret_cast<float4*>(dst) =
              make_float4(yt[tb][0], yt[tb][1], yt[tb][2], yt[tb][3]);
      }
      norm_partial(n, yt);
      if (n >= 2) norm_gather(n - 2, true);
    }
    if constexpr (NBUF == 1) {
      __syncthreads();  // every wave is done with this chunk's tiles
      stage(0, 0, NPF);
    } else {
      stage(cur ^ 1, kHalf ? NH : 0, NPF);
    }
    __syncthreads();
  }

  if constexpr (kNorm) {
    // The last chunks: N−3 has its rstd and values loaded, N−2 its sums
    // published, N−1 its per-wave partials.
    if (p.N >= 3) norm_finish(p.N - 3);
    if (p.N >= 2) norm_gather(p.N - 2, false);
    norm_publish(p.N - 1);
    __syncthreads();
    if (p.N >= 2) {
      norm_start(p.N - 2);
      norm_finish(p.N - 2);
    }
    norm_gather(p.N - 1, false);
    __syncthreads();
    norm_start(p.N - 1);
    norm_finish(p.N - 1);
  }

  float* sout = p.s_out + size_t(bh) * K * p.V + jl;
  int ld = p.V;
  if constexpr (SEG == 1) {
    sout = trans ? p.seg_m + size_t(bh) * K * K + (jl - p.V) : p.seg_h + size_t(bh) * K * p.V + jl;
    ld = trans ? K : p.V;
  } else if constexpr (SEG == 2) {
    // only the last segment's end state leaves the call
    if (b % p.seg_p != p.seg_p - 1) return;
    sout = p.seg_final + (size_t(b / p.seg_p) * p.H + h) * K * p.V + jl;
  }
#pragma unroll
  for (int rb = 0; rb < RBK; ++rb)
#pragma unroll
    for (int r = 0; r < 4; ++r) sout[size_t(16 * rb + 4 * q4 + r) * ld] = S[rb][r];
}

}  // namespace
}  // namespace dn
