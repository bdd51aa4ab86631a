// T = (I + A)⁻¹ for a 64×64 strictly lower A in LDS (fp32), by blocked forward
// substitution on four 64-lane waves: each wave inverts one 16×16 diagonal
// block by column elimination, then two doubling merges on fp32 MFMA complete
// the lower blocks. L³/3 flops, where the reference's ladder
// (src/delta/tri/prim.rs:28-51) spends 24·L³.
#pragma once

#include "mfma_util.hpp"

namespace dn {

constexpr int kWyL = 64;  // chunk length of the MFMA paths

// Value of lane `SRC` of each group of four lanes, to the whole group (DPP
// quad_perm).
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

// T's diagonal 16×16 block `wave` of T = (I + A)⁻¹ (A strict lower, fp32 in
// LDS) by column elimination; one wave per block. Lane (c, g) holds rows g,
// g+4, g+8, g+12 of column c; step k₂ broadcasts x[k₂] inside the lane quad
// (DPP) and updates the rows below it.
__device__ inline void diag_inverse(const float (*A)[kWyL + 1], float (*Tm)[kWyL + 1], int wave,
                                    int lane) {
  const int base = 16 * wave, c = lane >> 2, g = lane & 3;
  float x[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) x[j] = (4 * j + g == c) ? 1.f : 0.f;
  // Multipliers A[i][k₂] for i > k₂ (zero otherwise), read a batch of five
  // columns ahead of their use (20 registers rather than 60).
  float mul[2][5][4];
  auto fetch = [&](int batch, float (&m)[5][4]) {
#pragma unroll
    for (int u = 0; u < 5; ++u)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const int k2 = 5 * batch + u, i = 4 * j + g;
        m[u][j] = (4 * j + 3 > k2 && i > k2) ? A[base + i][base + k2] : 0.f;
      }
  };
  fetch(0, mul[0]);
#pragma unroll
  for (int batch = 0; batch < 3; ++batch) {
    if (batch + 1 < 3) fetch(batch + 1, mul[(batch + 1) & 1]);
#pragma unroll
    for (int u = 0; u < 5; ++u) {
      const int k2 = 5 * batch + u;
      const float xk = quad_bcast(x[k2 >> 2], k2 & 3);
#pragma unroll
      for (int j = 0; j < 4; ++j)
        if (4 * j + 3 > k2) x[j] -= mul[batch & 1][u][j] * xk;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) Tm[base + 4 * j + g][base + c] = x[j];
}

// The two doubling merges that complete T from its diagonal blocks, in three
// steps that waves 0..3 run with a barrier between consecutive steps (and
// after diag_inverse before the first). They neither read nor write T above
// its block diagonal. They run on v_mfma_f32_16x16x4_f32
// (exact fp32 products): lane l holds A[l%16][l/16] and B[l/16][l%16] of a
// 16×4 · 4×16 step, and D[4(l/16)+r][l%16]. Full-block sums are exact: the
// triangular factors hold zeros outside their triangles.
//
// Step 1 (waves 0 and 1), 16 → 32: T₁₀ = −T₁₁ A₁₀ T₀₀ for the two 32-blocks.
// Each wave writes and reads back only its own rows of Xs; a wave's LDS
// accesses complete in order, so no barrier is needed between them.
// Xs: 32 rows of at least 16 floats (row pitch XP).
template <int XP>
__device__ inline void merge_step1(const float (*A)[kWyL + 1], float (*Tm)[kWyL + 1],
                                   float (*Xs)[XP], int wave, int lane) {
  const int m16 = lane & 15, g4 = lane >> 4;
  if (wave >= 2) return;
  const int r0 = 32 * wave + 16, c0 = 32 * wave;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4)
    acc = mfma_f32(A[r0 + m16][c0 + 4 * s4 + g4], Tm[c0 + 4 * s4 + g4][c0 + m16], acc);
#pragma unroll
  for (int r = 0; r < 4; ++r) Xs[16 * wave + 4 * g4 + r][m16] = acc[r];
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront", "local");
  acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s4 = 0; s4 < 4; ++s4)
    acc = mfma_f32(Tm[r0 + m16][r0 + 4 * s4 + g4], Xs[16 * wave + 4 * s4 + g4][m16], acc);
#pragma unroll
  for (int r = 0; r < 4; ++r) Tm[r0 + 4 * g4 + r][c0 + m16] = -acc[r];
}

// Step 2 (waves 0..3), 32 → 64, first half: Xs = A[32:,:32]·T[:32,:32]; wave
// w owns output tile (w/2, w%2). The last read of A. T's block above the
// diagonal is zero and not read: output column block 1 starts at k = 16.
__device__ inline void merge_step2(const float (*A)[kWyL + 1], const float (*Tm)[kWyL + 1],
                                   float (*Xs)[kWyL / 2 + 1], int wave, int lane) {
  const int m16 = lane & 15, g4 = lane >> 4;
  if (wave >= 4) return;
  const int ti = wave >> 1, tj = wave & 1;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s4 = 0; s4 < 8; ++s4)
    if (s4 >= 4 * tj)
      acc = mfma_f32(A[32 + 16 * ti + m16][4 * s4 + g4], Tm[4 * s4 + g4][16 * tj + m16], acc);
#pragma unroll
  for (int r = 0; r < 4; ++r) Xs[16 * ti + 4 * g4 + r][16 * tj + m16] = acc[r];
}

// Step 3 (waves 0..3): T[32:,:32] = −T[32:,32:]·Xs. Row block 2 of T is zero
// past its diagonal block (k ≥ 48) and not read.
__device__ inline void merge_step3(float (*Tm)[kWyL + 1], const float (*Xs)[kWyL / 2 + 1],
                                   int wave, int lane) {
  const int m16 = lane & 15, g4 = lane >> 4;
  if (wave >= 4) return;
  const int ti = wave >> 1, tj = wave & 1;
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int s4 = 0; s4 < 8; ++s4)
    if (s4 < 4 + 4 * ti)
      acc = mfma_f32(Tm[32 + 16 * ti + m16][32 + 4 * s4 + g4], Xs[4 * s4 + g4][16 * tj + m16],
                     acc);
#pragma unroll
  for (int r = 0; r < 4; ++r) Tm[32 + 16 * ti + 4 * g4 + r][16 * tj + m16] = -acc[r];
}

// Steps 2 and 3 as one step of waves 0..3 with no barrier inside (after
// step 1 and a barrier): wave w = 2·ti + tj forms the products it needs,
// Xs(l) = A[32+16l…][:32]·T[:32][16tj…] for l ≤ ti, in its own scratch Xw
// (two 16×16 fp32 tiles, read back only by the wave itself), then
// T[32+16ti…][16tj…] = −Σ_{l≤ti} T[32+16ti…][32+16l…]·Xs(l). T above its
// block diagonal is not read. The last read of A.
__device__ inline void merge_steps23(const float (*A)[kWyL + 1], float (*Tm)[kWyL + 1],
                                     float (*Xw)[17], int wave, int lane) {
  if (wave >= 4) return;
  const int m16 = lane & 15, g4 = lane >> 4;
  const int ti = wave >> 1, tj = wave & 1;
  f32x4 xs[2];
#pragma unroll
  for (int l = 0; l < 2; ++l) {
    xs[l] = f32x4{0.f, 0.f, 0.f, 0.f};
    if (l <= ti) {
#pragma unroll
      for (int s4 = 0; s4 < 8; ++s4)
        if (s4 >= 4 * tj)
          xs[l] = mfma_f32(A[32 + 16 * l + m16][4 * s4 + g4], Tm[4 * s4 + g4][16 * tj + m16],
                           xs[l]);
    }
  }
#pragma unroll
  for (int l = 0; l < 2; ++l)
    if (l <= ti) {
#pragma unroll
      for (int r = 0; r < 4; ++r) Xw[16 * l + 4 * g4 + r][m16] = xs[l][r];
    }
  __builtin_amdgcn_fence(__ATOMIC_ACQ_REL, "wavefront", "local");
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int l = 0; l < 2; ++l)
    if (l <= ti) {
#pragma unroll
      for (int s4 = 0; s4 < 4; ++s4)
        acc = mfma_f32(Tm[32 + 16 * ti + m16][32 + 16 * l + 4 * s4 + g4],
                       Xw[16 * l + 4 * s4 + g4][m16], acc);
    }
#pragma unroll
  for (int r = 0; r < 4; ++r) Tm[32 + 16 * ti + 4 * g4 + r][16 * tj + m16] = -acc[r];
}

// The three steps with `sync` (a barrier of the calling waves) between them
// and on return.
template <class Sync>
__device__ inline void merge_T(const float (*A)[kWyL + 1], float (*Tm)[kWyL + 1],
                               float (*Xs)[kWyL / 2 + 1], int wave, int lane, Sync sync) {
  merge_step1(A, Tm, Xs, wave, lane);
  sync();
  merge_step2(A, Tm, Xs, wave, lane);
  sync();
  merge_step3(Tm, Xs, wave, lane);
  sync();
}

}  // namespace dn
