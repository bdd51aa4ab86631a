// Helpers shared by the bf16-MFMA kernels (gfx950, 64-lane waves).
//
// v_mfma_f32_16x16x32_bf16: lane l supplies A[l%16][8(l/16) .. 8(l/16)+7] and
// B[8(l/16) .. 8(l/16)+7][l%16] and receives D[4(l/16)+r][l%16], r = 0..3.
// A and B fragments share one layout, so C = A·Bᵀ reads both operands from
// tiles stored with the contraction index fastest ("NT" products).
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace dn {

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;

__device__ inline f32x4 mfma16(const bf16x8& a, const bf16x8& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}
__device__ inline f32x4 mfma16(const uint4& a, const uint4& b, const f32x4& c) {
  return mfma16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c);
}

__device__ inline bf16x8 ld8(const uint16_t* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ inline uint4 ld8u(const uint16_t* p) { return *reinterpret_cast<const uint4*>(p); }

// Two floats → packed bf16 (round to nearest even), one v_cvt_pk_bf16_f32.
__device__ inline uint32_t pk_bf16(float a, float b) {
  const bf16x2 v = {(__bf16)a, (__bf16)b};
  return __builtin_bit_cast(uint32_t, v);
}
// Low / high bf16 of a packed pair, as floats.
__device__ inline float lo_f(uint32_t u) { return __uint_as_float(u << 16); }
__device__ inline float hi_f(uint32_t u) { return __uint_as_float(u & 0xffff0000u); }

// Eight floats → bf16 hi parts and the bf16 lo parts of the remainders
// (hi + lo carries ~16 significant bits).
__device__ inline void split8(const float* f, uint4& h, uint4& l) {
  h = make_uint4(pk_bf16(f[0], f[1]), pk_bf16(f[2], f[3]), pk_bf16(f[4], f[5]),
                 pk_bf16(f[6], f[7]));
  l = make_uint4(pk_bf16(f[0] - lo_f(h.x), f[1] - hi_f(h.x)),
                 pk_bf16(f[2] - lo_f(h.y), f[3] - hi_f(h.y)),
                 pk_bf16(f[4] - lo_f(h.z), f[5] - hi_f(h.z)),
                 pk_bf16(f[6] - lo_f(h.w), f[7] - hi_f(h.w)));
}
__device__ inline void unpack8(const uint4& u, float* f) {
  f[0] = lo_f(u.x); f[1] = hi_f(u.x); f[2] = lo_f(u.y); f[3] = hi_f(u.y);
  f[4] = lo_f(u.z); f[5] = hi_f(u.z); f[6] = lo_f(u.w); f[7] = hi_f(u.w);
}

__device__ inline f32x4 mfma_f32(float a, float b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// Operand tiles in LDS. Within every 32-deep k-step the contraction index
// may be stored permuted so that the 8 values an MFMA lane supplies
// (positions 8q..8q+7 of the step) are rows 4q..4q+3 and 16+4q..16+4q+3 of
// it — exactly the rows a 16×16 accumulator lane holds in two vertically
// adjacent tiles. Accumulator tiles thereby become MFMA operands in place,
// with no LDS round trip.
__device__ inline int perm_pos(int k) {
  const int m = k & 31;
  return (k & ~31) + 8 * ((m & 15) >> 2) + 4 * (m >> 4) + (m & 3);
}
// A workgroup barrier that orders LDS only: this wave's LDS accesses have
// completed (lgkmcnt 0) when it arrives, and the compiler moves no memory
// access across it. __syncthreads() also waits for every global load and
// store in flight (vmcnt 0), so loads issued ahead of a barrier for use after
// it would be waited for at the barrier; here they are waited for at their
// first use. For barriers between waves that communicate through LDS only,
// and for HBM → LDS copies that are waited for explicitly.
__device__ inline void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Element (row, pos) of a tile with COLS bf16 per row; 16-byte chunks are
// XOR-swizzled by row so the 16 rows of a fragment read land in 16 distinct
// bank slots.
template <int COLS>
__device__ inline int tile_at(int row, int pos) {
  const int sw = COLS >= 128 ? (row & 15) : ((row >> 1) & 7);
  return row * COLS + (((pos >> 3) ^ sw) << 3) + (pos & 7);
}

// Two vertically adjacent 16×16 accumulator tiles → one bf16 operand
// fragment of the permuted layout (hi part, and optionally the lo part).
__device__ inline uint4 frag_hi(const f32x4& a, const f32x4& b) {
  return make_uint4(pk_bf16(a[0], a[1]), pk_bf16(a[2], a[3]), pk_bf16(b[0], b[1]),
                    pk_bf16(b[2], b[3]));
}
__device__ inline uint4 frag_lo(const f32x4& a, const f32x4& b, const uint4& h) {
  return make_uint4(pk_bf16(a[0] - lo_f(h.x), a[1] - hi_f(h.x)),
                    pk_bf16(a[2] - lo_f(h.y), a[3] - hi_f(h.y)),
                    pk_bf16(b[0] - lo_f(h.z), b[1] - hi_f(h.z)),
                    pk_bf16(b[2] - lo_f(h.w), b[3] - hi_f(h.w)));
}

// A 64×64 triangular tile times a 64-row operand, as MFMA steps over 4 row
// blocks of 16 and 2 k-steps of 32: six of the eight (row block, k-step)
// pairs are nonzero. Lower triangular (T, attn): row blocks 0 and 1 have no
// k-step 1. Step s of the six, in row-block order.
constexpr int kTriSteps = 6;
__host__ __device__ constexpr int tril_tb(int s) { return s < 2 ? s : 2 + ((s - 2) >> 1); }
__host__ __device__ constexpr int tril_kk(int s) { return s < 2 ? 0 : (s - 2) & 1; }
__host__ __device__ constexpr int tril_step(int tb, int kk) { return tb < 2 ? tb : 2 * tb - 2 + kk; }

// The forward's T, T lo and attn of a chunk-head in HBM, packed: each
// lower-triangular 64×64 tile as its six nonzero 16×32 blocks (in step order,
// row-major inside a block), the three tiles back to back. The two blocks
// above the diagonal band are never stored or read: a quarter less tile
// traffic between the intra kernel and the scan.
constexpr int kTriBlk = 16 * 32;
constexpr int kTriPacked = kTriSteps * kTriBlk;  // elements per packed tile
constexpr int kTriTrio = 3 * kTriPacked;         // per chunk-head
// Whether the per-head forward's intra kernel and scan pass the tiles
// packed: not for the backward's recompute (its transposing reads take full
// tiles), nor at head_k_dim 256, whose single-buffered scan ran slower on
// packed tiles (B=8 T=4096 H=16 dv=256: 0.68 → 0.86 ms).
__host__ __device__ constexpr bool tri_packed(int K, bool backward) {
  return !backward && K <= 128;
}

}  // namespace dn
